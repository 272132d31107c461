// sfg_attention.hip -- GQA attention for gfx950.
//
//  * attn_prefill_rows_kernel: online softmax (attention_compiler.cpp:286-377),
//    one wave per query row, 64 keys per step (one per lane), values
//    accumulated with the wave owning the head dimension (up to 256): the
//    fp32 path, and bf16 head dims the MFMA kernels do not lower.
//  * attn_prefill_bf16_kernel: IO-aware flash prefill on v_mfma_f32_32x32x16_bf16.
//    A workgroup owns 128 query rows of one (batch, head); each wave 32 rows.
//    Scores are formed transposed, S^T = K Q^T, so lane l owns query row
//    (l & 31) for 32 of every 64 keys (lane l ^ 32 has the other 32): the row
//    max / sum need one cross-lane step, and the output is accumulated
//    transposed, O^T = V^T P^T, so the online-softmax rescale is a per-lane
//    scalar.  K and V^T tiles of 64 keys are staged through padded LDS;
//    causal tiles beyond a wave's last row are skipped.
//  * attn_decode_split_kernel + attn_decode_combine_kernel: paged Split-KV
//    decode (attention_compiler.cpp:244-285 split, 132-145 merge_online;
//    next_milestones.cpp:137-184 page walk).  A workgroup owns (sequence,
//    kv_head, split) and serves the whole GQA group, so each K/V byte is read
//    once; scores and the value product run on MFMA (see below), pages are
//    double-buffered in registers, waves merge in LDS, splits merge in a
//    second small kernel.
#include <cstdlib>
#include <type_traits>

#include "sfg_kernels.hpp"

namespace sfg {

// ===========================================================================
// Row-per-wave prefill, any head_dim up to kRowMaxD: the fp32 path, and bf16
// shapes the MFMA kernels do not lower (head_dim other than 64 / 128).
// ===========================================================================
constexpr int kRowMaxD = 256;

template <typename InT>
__device__ __forceinline__ float in_f32(const InT* p, int64_t i) {
    if constexpr (sizeof(InT) == 4) return p[i];
    else return bf16_to_f32(p[i]);
}

// One wave per query row, the workgroup's four rows (consecutive rows of one
// head) sharing each 64-key chunk of K and V, which the workgroup stages into
// LDS with coalesced loads (K rows padded to D + 1 floats, so the 64 lanes
// reading one key row each touch distinct banks).  Lane j then scores key j
// of the chunk with one sequential fp32 FMA chain over the head dimension, and
// the wave accumulates p V with lane d owning dims d, d + 64, ... (online
// softmax, attention_compiler.cpp:102-112).
template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void attn_prefill_rows_kernel(
    const InT* __restrict__ q, const InT* __restrict__ k, const InT* __restrict__ v,
    OutT* __restrict__ out, int q_heads, int kv_heads, int seq_q, int seq_kv, int head_dim,
    int causal, float scale) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int q0 = blockIdx.x * 4;
    const int qi = q0 + wave;
    const int h = blockIdx.y, b = blockIdx.z;
    __shared__ float sq[4][kRowMaxD];
    __shared__ float sK[64 * (kRowMaxD + 1)];
    __shared__ float sV[64 * kRowMaxD];
    const bool live = qi < seq_q;
    const int kvh = h * kv_heads / q_heads;
    if (live) {
        const InT* qr = q + ((static_cast<int64_t>(b) * q_heads + h) * seq_q + qi) * head_dim;
        for (int d = lane; d < head_dim; d += 64) sq[wave][d] = in_f32(qr, d);
    }
    const InT* kb = k + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * head_dim;
    const InT* vb = v + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * head_dim;
    const int limit = causal ? (seq_kv - seq_q + qi) : (seq_kv - 1);
    // keys the workgroup's last live row attends to
    const int q_last = min(q0 + 3, seq_q - 1);
    const int block_limit = min(causal ? (seq_kv - seq_q + q_last) : (seq_kv - 1), seq_kv - 1);
    const int kstride = head_dim + 1;
    const float inv_d = 1.0f / static_cast<float>(head_dim);
    float m = -INFINITY, l = 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // dims lane + 64 r
    for (int base = 0; base <= block_limit; base += 64) {
        const int nkeys = min(64, block_limit - base + 1);
        const int total = nkeys * head_dim;
        __syncthreads();  // the previous chunk's reads are done
        // eight loads of each operand in flight per thread: the loads past
        // the chunk re-read its last element (no branch around a load) and
        // are not stored
        for (int e0 = threadIdx.x; e0 < total; e0 += 256 * 8) {
            float kv[8], vv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t src = static_cast<int64_t>(base) * head_dim + min(e0 + 256 * i, total - 1);
                kv[i] = in_f32(kb, src);
                vv[i] = in_f32(vb, src);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = e0 + 256 * i;
                if (e < total) {
                    // row = e / head_dim: (e + 0.5) / D stays at least 0.5 / D
                    // away from an integer, far beyond float error for e < 2^15
                    const int row = static_cast<int>((static_cast<float>(e) + 0.5f) * inv_d);
                    sK[e + row] = kv[i];  // row * (D + 1) + col
                    sV[e] = vv[i];
                }
            }
        }
        __syncthreads();
        if (!live || base > limit) continue;
        const int j = base + lane;
        float s = -INFINITY;
        if (j <= limit && j < seq_kv) {
            const float* kr = sK + lane * kstride;
            float dot = 0.f;
            // eight steps' operands read before their FMAs (same chain order)
            int d = 0;
            for (; d + 8 <= head_dim; d += 8) {
                float qv[8], kv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    qv[i] = sq[wave][d + i];
                    kv[i] = kr[d + i];
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) dot = fmaf(qv[i], kv[i], dot);
            }
            for (; d < head_dim; ++d) dot = fmaf(sq[wave][d], kr[d], dot);
            s = dot * scale;
        }
        const float mx = wave_max(s);
        const float m_new = fmaxf(m, mx);
        const float alpha = (m == -INFINITY) ? 0.f : expf(m - m_new);
        const float p = (s == -INFINITY) ? 0.f : expf(s - m_new);
        l = l * alpha + wave_sum(p);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= alpha;
        const int count = min(64, min(limit, seq_kv - 1) - base + 1);
        int t = 0;
        for (; t + 8 <= count; t += 8) {
            float pt[8], vv[8][4];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pt[i] = lane_bcast(p, t + i);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    vv[i][r] = lane + 64 * r < head_dim ? sV[(t + i) * head_dim + lane + 64 * r] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (lane + 64 * r < head_dim) acc[r] = fmaf(pt[i], vv[i][r], acc[r]);
        }
        for (; t < count; ++t) {
            const float pt = lane_bcast(p, t);
            const float* vr = sV + t * head_dim;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (lane + 64 * r < head_dim) acc[r] = fmaf(pt, vr[lane + 64 * r], acc[r]);
        }
        m = m_new;
    }
    if (!live) return;
    const int64_t row = static_cast<int64_t>(b) * seq_q + qi;
    OutT* orow = out + row * (static_cast<int64_t>(q_heads) * head_dim) + h * head_dim;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int d = lane + 64 * r;
        if (d < head_dim) {
            const float o = acc[r] / l;
            if constexpr (sizeof(OutT) == 4) orow[d] = o; else orow[d] = f32_to_bf16(o);
        }
    }
}

template <typename InT>
static void launch_prefill_rows(const InT* q, const InT* k, const InT* v, void* out, int out_dtype,
                                int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                                int64_t seq_kv, int64_t head_dim, int causal, float scale,
                                hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((seq_q + 3) / 4), static_cast<unsigned>(q_heads),
                    static_cast<unsigned>(batch));
    if (out_dtype == SFG_F32)
        attn_prefill_rows_kernel<InT, float><<<grid, 256, 0, stream>>>(
            q, k, v, static_cast<float*>(out), q_heads, kv_heads, seq_q, seq_kv, head_dim, causal,
            scale);
    else
        attn_prefill_rows_kernel<InT, uint16_t><<<grid, 256, 0, stream>>>(
            q, k, v, static_cast<uint16_t*>(out), q_heads, kv_heads, seq_q, seq_kv, head_dim,
            causal, scale);
}

int launch_attn_prefill_f32(const float* q, const float* k, const float* v, void* out,
                            int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                            int64_t seq_q, int64_t seq_kv, int64_t head_dim, int causal,
                            float scale, hipStream_t stream) {
    if (head_dim > kRowMaxD) return SFG_ERR_UNSUPPORTED;
    launch_prefill_rows(q, k, v, out, out_dtype, batch, q_heads, kv_heads, seq_q, seq_kv, head_dim,
                        causal, scale, stream);
    return SFG_OK;
}

// ===========================================================================
// bf16 MFMA flash prefill, head_dim 128 or 64.
// ===========================================================================
constexpr int kFaD = 128;
constexpr int kFaBM = 128;          // query rows per workgroup
constexpr int kFaBN = 64;           // keys per tile
constexpr int kVRow = kFaBN + 8;    // padded V^T row

template <typename OutT, int kD>
__global__ __launch_bounds__(256) void attn_prefill_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, OutT* __restrict__ out, int q_heads, int kv_heads,
    int seq_q, int seq_kv, int causal, float scale_log2) {
    static_assert(kD == 64 || kD == 128, "head_dim 64 or 128");
    constexpr int kKRow = kD + 8;       // padded K row (bf16 elements)
    constexpr int kQs = kD / 16;        // k-steps of S^T = K Q^T
    constexpr int kOd = kD / 32;        // 32-dim blocks of O^T
    constexpr int kChunks = kD / 8;     // 16-byte chunks per key row
    __shared__ __attribute__((aligned(16))) uint16_t sK[kFaBN * kKRow];
    __shared__ __attribute__((aligned(16))) uint16_t sVt[kD * kVRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int qblock = gridDim.x - 1 - blockIdx.x;  // heavy causal blocks first
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h * kv_heads / q_heads;
    const int offset = seq_kv - seq_q;              // causal alignment
    const int q0 = qblock * kFaBM;
    const int qw0 = q0 + wave * 32;
    const int my_q = qw0 + l32;

    // Q fragments (B operand of S^T = K Q^T): lane supplies row my_q,
    // d = 16 * step + 8 * half + [0, 8).
    bf16x8 qf[kQs];
    {
        const uint16_t* qr = q + ((static_cast<int64_t>(b) * q_heads + h) * seq_q + my_q) * kD;
#pragma unroll
        for (int s = 0; s < kQs; ++s) {
            uint4 val = make_uint4(0, 0, 0, 0);
            if (my_q < seq_q) val = *reinterpret_cast<const uint4*>(qr + s * 16 + half * 8);
            qf[s] = as_bf16x8(val);
        }
    }
    const uint16_t* kb = k + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * kD;
    const uint16_t* vb = v + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * kD;

    floatx16 acc_o[kOd];
#pragma unroll
    for (int i = 0; i < kOd; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[i][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int block_last_q = min(q0 + kFaBM, seq_q) - 1;
    const int kv_limit = causal ? min(seq_kv, block_last_q + offset + 1) : seq_kv;
    const int tiles = (kv_limit + kFaBN - 1) / kFaBN;
    const int wave_last_key = causal ? (min(qw0 + 31, seq_q - 1) + offset) : (seq_kv - 1);

    for (int t = 0; t < tiles; ++t) {
        const int kv0 = t * kFaBN;
        __syncthreads();
        // Stage K [64][D] and V^T [D][64]: 8 D 16-byte chunks each.
#pragma unroll
        for (int it = 0; it < kFaBN * kChunks / 256; ++it) {
            const int idx = tid + it * 256;
            const int key = idx / kChunks;
            const int chunk = (idx % kChunks) * 8;
            uint4 kv4 = make_uint4(0, 0, 0, 0), vv4 = make_uint4(0, 0, 0, 0);
            if (kv0 + key < seq_kv) {
                kv4 = *reinterpret_cast<const uint4*>(kb + static_cast<int64_t>(kv0 + key) * kD + chunk);
                vv4 = *reinterpret_cast<const uint4*>(vb + static_cast<int64_t>(kv0 + key) * kD + chunk);
            }
            *reinterpret_cast<uint4*>(&sK[key * kKRow + chunk]) = kv4;
            const uint16_t* ve = reinterpret_cast<const uint16_t*>(&vv4);
#pragma unroll
            for (int e = 0; e < 8; ++e) sVt[(chunk + e) * kVRow + key] = ve[e];
        }
        __syncthreads();
        if (kv0 > wave_last_key || qw0 >= seq_q) continue;

        // S^T sub-tiles: 2 x (32 keys x 32 queries).
        floatx16 s_acc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s_acc[j][r] = 0.f;
#pragma unroll
            for (int s = 0; s < kQs; ++s) {
                const bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &sK[(j * 32 + l32) * kKRow + s * 16 + half * 8]));
                s_acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], s_acc[j], 0, 0, 0);
            }
        }
        // Scale, mask, row max.  Element r of sub-tile j is key
        // kv0 + 32 j + 8 (r / 4) + 4 half + (r % 4), query my_q.
        const int my_limit = causal ? (my_q + offset) : (seq_kv - 1);
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kv0 + j * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                float sv = s_acc[j][r] * scale_log2;
                if (key > my_limit || key >= seq_kv) sv = -INFINITY;
                s_acc[j][r] = sv;
                tmax = fmaxf(tmax, sv);
            }
        tmax = xor32_max(tmax);
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
        float psum = 0.f;
        bf16x8 pf[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float pv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float sv = s_acc[j][r];
                pv[r] = (sv == -INFINITY) ? 0.f : fast_exp2(sv - m_new);
                psum += pv[r];
            }
            pf[j][0] = as_bf16x8(f32x8_to_bf16x8(&pv[0]));
            pf[j][1] = as_bf16x8(f32x8_to_bf16x8(&pv[8]));
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < kOd; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc_o[i][r] *= alpha;
        // O^T[d][q] += V^T[d][key] P^T[key][q].  MFMA k index (8 half + jj)
        // maps to key 32 j + 16 t + 4 half + (jj < 4 ? jj : 4 + jj), the keys
        // this lane holds in P, so V^T is read at the same two 4-key runs.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int kbase = j * 32 + tt * 16 + 4 * half;
#pragma unroll
                for (int i = 0; i < kOd; ++i) {
                    const int d = i * 32 + l32;
                    const uint2 lo = *reinterpret_cast<const uint2*>(&sVt[d * kVRow + kbase]);
                    const uint2 hi = *reinterpret_cast<const uint2*>(&sVt[d * kVRow + kbase + 8]);
                    const uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    acc_o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(vv), pf[j][tt],
                                                                      acc_o[i], 0, 0, 0);
                }
            }
    }
    if (my_q >= seq_q) return;
    const float l_total = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = 1.0f / l_total;
    // O^T layout: lane holds query my_q, dims 32 i + 8 (r / 4) + 4 half + (r % 4).
    const int64_t row = static_cast<int64_t>(b) * seq_q + my_q;
    OutT* orow = out + row * (static_cast<int64_t>(q_heads) * kD) + h * kD;
#pragma unroll
    for (int i = 0; i < kOd; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = i * 32 + 8 * c + 4 * half;
            const float o0 = acc_o[i][4 * c + 0] * inv, o1 = acc_o[i][4 * c + 1] * inv;
            const float o2 = acc_o[i][4 * c + 2] * inv, o3 = acc_o[i][4 * c + 3] * inv;
            if constexpr (sizeof(OutT) == 4) {
                *reinterpret_cast<float4*>(orow + d) = make_float4(o0, o1, o2, o3);
            } else {
                uint2 pk;
                pk.x = pack_bf16x2(o0, o1);
                pk.y = pack_bf16x2(o2, o3);
                *reinterpret_cast<uint2*>(orow + d) = pk;
            }
        }
}

int launch_attn_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, void* out,
                             int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t seq_q, int64_t seq_kv, int64_t head_dim, int causal,
                             float scale, hipStream_t stream) {
    if (head_dim != 128 && head_dim != 64) {
        // other head dims: the row-per-wave kernel on the bf16 operands
        if (head_dim > kRowMaxD) return SFG_ERR_UNSUPPORTED;
        launch_prefill_rows(q, k, v, out, out_dtype, batch, q_heads, kv_heads, seq_q, seq_kv,
                            head_dim, causal, scale, stream);
        return SFG_OK;
    }
    const float scale_log2 = scale * kLog2e;
    const dim3 grid(static_cast<unsigned>((seq_q + kFaBM - 1) / kFaBM),
                    static_cast<unsigned>(q_heads), static_cast<unsigned>(batch));
    const int qh = static_cast<int>(q_heads), kvh = static_cast<int>(kv_heads);
    const int sq = static_cast<int>(seq_q), skv = static_cast<int>(seq_kv);
    if (head_dim == 128) {
        if (out_dtype == SFG_F32)
            attn_prefill_bf16_kernel<float, 128><<<grid, 256, 0, stream>>>(
                q, k, v, static_cast<float*>(out), qh, kvh, sq, skv, causal, scale_log2);
        else
            attn_prefill_bf16_kernel<uint16_t, 128><<<grid, 256, 0, stream>>>(
                q, k, v, static_cast<uint16_t*>(out), qh, kvh, sq, skv, causal, scale_log2);
    } else {
        if (out_dtype == SFG_F32)
            attn_prefill_bf16_kernel<float, 64><<<grid, 256, 0, stream>>>(
                q, k, v, static_cast<float*>(out), qh, kvh, sq, skv, causal, scale_log2);
        else
            attn_prefill_bf16_kernel<uint16_t, 64><<<grid, 256, 0, stream>>>(
                q, k, v, static_cast<uint16_t*>(out), qh, kvh, sq, skv, causal, scale_log2);
    }
    return SFG_OK;
}

// ===========================================================================
// bf16 flash prefill over a transposed value tensor, head_dim 128.
//
// Inputs: Q [B][Hq][Sq][128], K [B][Hkv][Skv][128], V^T [B][Hkv][128][ld_vt]
// (keys in [Skv, ld_vt) are zero; ld_vt is a multiple of 64 >= Skv).
// A workgroup of WAVES waves owns 32 * WAVES query rows of one (batch, head);
// a wave owns 32 rows.  Per tile of 64 keys:
//   S^T[64 keys][32 q] = K Q^T      2 x 8 mfma_f32_32x32x16_bf16 (Q in VGPRs)
//   O^T[128 d][32 q] += V^T P^T     4 x 4 mfma_f32_32x32x16_bf16
// K and V^T tiles go global -> LDS directly (LDS DMA), in two stages for four
// waves (the next tile in flight while the current one is multiplied) and
// three for eight (the next two).
// Key order: the K fragment of lane l is key row swap23(l & 31) of its 32-key
// block (bits 2 and 3 of the index exchanged), so accumulator register r of
// lane l holds key 16 (r / 8) + 8 (l / 32) + r % 8 -- eight consecutive keys
// per MFMA k-step, which is the P^T operand layout and a single 16-byte V^T
// fragment read.  LDS slots are XOR-swizzled by row so fragment reads of 16
// consecutive lanes touch 16 distinct 16-byte slots.
// Online softmax in the exp2 domain with a lazy rescale: a row keeps its
// running max until a tile's max exceeds it by more than 8 (p <= 2^8), so the
// O^T rescale runs only when some row of the wave moved that far.
// Work order: consecutive workgroup ids go to the XCDs in turn; each XCD
// gets a contiguous run of (batch, kv_head) groups -- the Q heads sharing one
// K/V stay in one L2 -- and within a group the longest causal blocks first.
// ===========================================================================
constexpr int kFa2BN = 64;

struct Fa2Args {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* vt;
    void* out;
    int out_f32;
    int q_heads, kv_heads, seq_q, seq_kv, ld_vt, causal, nqb;
    float scale_log2;
    int xcds;
};

__device__ __forceinline__ int swap23(int i) {
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_prefill_fa2_kernel(Fa2Args p) {
    constexpr int BM = WAVES * 32;
    constexpr int kBlk = 16 / WAVES;  // 1 KB blocks of K (and of V^T) per wave per tile
    // Four waves: two stages (two workgroups per CU); eight waves: three
    // stages (96 KB, one workgroup per CU), the next two tiles in flight.
    constexpr int kStages = WAVES == 8 ? 3 : 2;
    constexpr int kStage2 = kStages == 3 ? kFa2BN * kFaD : 8;
    __shared__ __attribute__((aligned(1024))) uint16_t sK0[kFa2BN * kFaD];
    __shared__ __attribute__((aligned(1024))) uint16_t sK1[kFa2BN * kFaD];
    __shared__ __attribute__((aligned(1024))) uint16_t sK2[kStage2];
    __shared__ __attribute__((aligned(1024))) uint16_t sV0[kFaD * kFa2BN];
    __shared__ __attribute__((aligned(1024))) uint16_t sV1[kFaD * kFa2BN];
    __shared__ __attribute__((aligned(1024))) uint16_t sV2[kStage2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hl = lane >> 5;
    const int l32 = lane & 31;

    // --- work item -------------------------------------------------------
    const int G = p.q_heads / p.kv_heads;
    const int total = static_cast<int>(gridDim.x);
    const int bid = static_cast<int>(blockIdx.x);
    const int x = p.xcds;
    const int full = total - total % x;
    const int L = bid < full ? (bid % x) * (full / x) + bid / x : bid;
    const int per_group = p.nqb * G;
    const int grp = L / per_group;
    const int rem = L - grp * per_group;
    const int qblock = p.nqb - 1 - rem / G;
    const int b = grp / p.kv_heads, kvh = grp - b * p.kv_heads;
    const int h = kvh * G + rem % G;

    const int offset = p.seq_kv - p.seq_q;
    const int q0 = qblock * BM;
    const int qw0 = q0 + wave * 32;
    const int my_q = qw0 + l32;

    // Q^T fragments: lane supplies query my_q, dims 16 s + 8 hl + [0, 8).
    bf16x8 qf[8];
    {
        const int qrow = min(my_q, p.seq_q - 1);
        const uint16_t* qr = p.q + ((static_cast<int64_t>(b) * p.q_heads + h) * p.seq_q + qrow) * kFaD;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(qr + s * 16 + hl * 8));
    }
    const uint16_t* kb = p.k + (static_cast<int64_t>(b) * p.kv_heads + kvh) * p.seq_kv * kFaD;
    const uint16_t* vtb = p.vt + (static_cast<int64_t>(b) * p.kv_heads + kvh) * kFaD * p.ld_vt;

    const int block_last_q = min(q0 + BM, p.seq_q) - 1;
    const int kv_limit = p.causal ? min(p.seq_kv, block_last_q + offset + 1) : p.seq_kv;
    const int tiles = (kv_limit + kFa2BN - 1) / kFa2BN;
    const int wave_last_key = p.causal ? (min(qw0 + 31, p.seq_q - 1) + offset) : (p.seq_kv - 1);
    const int wave_first_limit = p.causal ? (qw0 + offset) : (p.seq_kv - 1);
    const bool wave_live = qw0 < p.seq_q;

    // --- loads: K block i = rows 4 i + (lane >> 4), slot lane & 15 holds
    // chunk slot ^ swap23(row & 15); V^T block i = dims 8 i + (lane >> 3),
    // slot lane & 7 holds chunk slot ^ (row & 7) ^ ((row >> 3) & 1).
    // Loads go through buffer resources over this (batch, kv_head)'s K rows
    // and V^T rows (byte offsets): key rows at or past seq_kv read as zeros
    // and are masked out of the scores.
    const buf_rsrc rk = make_rsrc(kb, static_cast<uint32_t>(p.seq_kv) * kFaD * 2);
    const buf_rsrc rv = make_rsrc(vtb, static_cast<uint32_t>(p.ld_vt) * kFaD * 2);
    uint32_t k_off[kBlk], v_off[kBlk];
#pragma unroll
    for (int n = 0; n < kBlk; ++n) {
        const int blk = wave * kBlk + n;
        const int row = 4 * blk + (lane >> 4);
        k_off[n] = static_cast<uint32_t>(row * kFaD + ((lane & 15) ^ swap23(row & 15)) * 8) * 2;
        const int d = 8 * blk + (lane >> 3);
        const int vch = (lane & 7) ^ (d & 7) ^ ((d >> 3) & 1);
        v_off[n] = static_cast<uint32_t>(d * p.ld_vt + vch * 8) * 2;
    }
    auto issue = [&](uint16_t* dk, uint16_t* dv, int kv0) {
#pragma unroll
        for (int n = 0; n < kBlk; ++n)
            lds_dma16_buf(rk, k_off[n] + static_cast<uint32_t>(kv0) * kFaD * 2, dk + (wave * kBlk + n) * 512);
#pragma unroll
        for (int n = 0; n < kBlk; ++n)
            lds_dma16_buf(rv, v_off[n] + static_cast<uint32_t>(kv0) * 2, dv + (wave * kBlk + n) * 512);
    };

    floatx16 acc_o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[i][r] = 0.f;
    float m_run = -INFINITY;  // running max, scaled (log2) units
    float l_run = 0.f;        // this lane's partial row sum
    const float c = p.scale_log2;
    const int my_limit = p.causal ? (my_q + offset) : (p.seq_kv - 1);

    // K fragment rows: key swap23(l32) of each 32-key block; slot chunk ^ (l32 & 15).
    const int kfrag = swap23(l32) * kFaD;
    const int kswz = l32 & 15;
    const int vswz = (l32 & 7) ^ ((l32 >> 3) & 1);

    auto compute = [&](const uint16_t* sK, const uint16_t* sV, int kv0) {
        if (!wave_live || kv0 > wave_last_key) return;
        floatx16 s[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[j][r] = 0.f;
#pragma unroll
            for (int st = 0; st < 8; ++st) {
                const bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &sK[j * 32 * kFaD + kfrag + (((2 * st + hl) ^ kswz) * 8)]));
                s[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[j], 0, 0, 0);
            }
        }
        // mask (only tiles crossing the diagonal or the end of the keys)
        if (kv0 + kFa2BN - 1 > wave_first_limit || kv0 + kFa2BN > p.seq_kv) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kv0 + 32 * j + 16 * (r >> 3) + 8 * hl + (r & 7);
                    if (key > my_limit || key >= p.seq_kv) s[j][r] = -INFINITY;
                }
        }
        float tmax = s[0][0];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[j][r]);
        tmax = xor32_max(tmax) * c;
        const bool upd = tmax > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(upd)) {
            const float m_new = upd ? tmax : m_run;
            const float alpha = upd ? fast_exp2(m_run - m_new) : 1.0f;
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc_o[i][r] *= alpha;
            m_run = m_new;
        }
        const float nm = -m_run;
        bf16x8 pf[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                float pv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    pv[e] = fast_exp2(fmaf(s[j][8 * t + e], c, nm));
                    l_run += pv[e];
                }
                uint4 pk;
                pk.x = cvt_pk_bf16(pv[0], pv[1]);
                pk.y = cvt_pk_bf16(pv[2], pv[3]);
                pk.z = cvt_pk_bf16(pv[4], pv[5]);
                pk.w = cvt_pk_bf16(pv[6], pv[7]);
                pf[j][t] = as_bf16x8(pk);
            }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int slot = ((4 * j + 2 * t + hl) ^ vswz) * 8;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bf16x8 vf = as_bf16x8(*reinterpret_cast<const uint4*>(
                        &sV[(32 * i + l32) * kFa2BN + slot]));
                    acc_o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j][t], acc_o[i], 0, 0, 0);
                }
            }
    };

    if constexpr (kStages == 2) {
        issue(sK0, sV0, 0);
        wait_vmem_all();
        __syncthreads();
        for (int t = 0; t < tiles; t += 2) {
            if (t + 1 < tiles) issue(sK1, sV1, (t + 1) * kFa2BN);
            compute(sK0, sV0, t * kFa2BN);
            wait_vmem_all();
            __syncthreads();
            if (t + 1 >= tiles) break;
            if (t + 2 < tiles) issue(sK0, sV0, (t + 2) * kFa2BN);
            compute(sK1, sV1, (t + 1) * kFa2BN);
            wait_vmem_all();
            __syncthreads();
        }
    } else {
        // Tile t issues tile t + 2 into the stage tile t - 1 used (retired by
        // the barrier that ended tile t - 1), then waits for its own loads of
        // tile t + 1 only (the 2 kBlk loads of tile t + 2 stay in flight).
        // Every tile issues one load group (past the end it re-fetches the
        // last tile into a stage nobody reads again), so the count is uniform.
        const int last = (tiles - 1) * kFa2BN;
        issue(sK0, sV0, 0);
        issue(sK1, sV1, min(kFa2BN, last));
        wait_vmem_lds<2 * kBlk>();
        barrier_no_fence();
        for (int t = 0; t < tiles; t += 3) {
            issue(sK2, sV2, min((t + 2) * kFa2BN, last));
            compute(sK0, sV0, t * kFa2BN);
            wait_vmem_lds<2 * kBlk>();
            barrier_no_fence();
            if (t + 1 >= tiles) break;
            issue(sK0, sV0, min((t + 3) * kFa2BN, last));
            compute(sK1, sV1, (t + 1) * kFa2BN);
            wait_vmem_lds<2 * kBlk>();
            barrier_no_fence();
            if (t + 2 >= tiles) break;
            issue(sK1, sV1, min((t + 4) * kFa2BN, last));
            compute(sK2, sV2, (t + 2) * kFa2BN);
            wait_vmem_lds<2 * kBlk>();
            barrier_no_fence();
        }
        wait_vmem_all();
    }

    if (my_q >= p.seq_q) return;
    const float l_total = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = 1.0f / l_total;
    // O^T layout: lane holds query my_q, dims 32 i + 8 (r / 4) + 4 hl + (r % 4).
    const int64_t row = static_cast<int64_t>(b) * p.seq_q + my_q;
    const int64_t obase = row * (static_cast<int64_t>(p.q_heads) * kFaD) + h * kFaD;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const int d = i * 32 + 8 * cc + 4 * hl;
            const float o0 = acc_o[i][4 * cc + 0] * inv, o1 = acc_o[i][4 * cc + 1] * inv;
            const float o2 = acc_o[i][4 * cc + 2] * inv, o3 = acc_o[i][4 * cc + 3] * inv;
            if (p.out_f32) {
                *reinterpret_cast<float4*>(static_cast<float*>(p.out) + obase + d) = make_float4(o0, o1, o2, o3);
            } else {
                uint2 pk;
                pk.x = pack_bf16x2(o0, o1);
                pk.y = pack_bf16x2(o2, o3);
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + obase + d) = pk;
            }
        }
}

int64_t attn_vt_ld(int64_t seq_kv) { return (seq_kv + kFa2BN - 1) / kFa2BN * kFa2BN; }

int launch_attn_prefill_vt(const uint16_t* q, const uint16_t* k, const uint16_t* vt, int64_t ld_vt,
                           void* out, int out_dtype, int64_t batch, int64_t q_heads,
                           int64_t kv_heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                           int causal, float scale, int waves_policy, hipStream_t stream) {
    if (head_dim != kFaD) return SFG_ERR_UNSUPPORTED;
    if (ld_vt % kFa2BN != 0 || ld_vt < seq_kv) return SFG_ERR_SHAPE;
    // Policy 0: eight waves (256 query rows, a three-stage K / V^T ring: two
    // tiles of load latency hidden instead of one) once that grid holds at
    // least four workgroups per CU; below that the 128-row blocks balance
    // the causal work better.  Same results either way.
    int waves = waves_policy;
    if (waves != 4 && waves != 8) {
        const int64_t grid8 = (seq_q + 255) / 256 * q_heads * batch;
        waves = grid8 >= 4 * static_cast<int64_t>(device_cus(stream)) ? 8 : 4;
    }
    const int bm = waves * 32;
    Fa2Args a{};
    a.q = q; a.k = k; a.vt = vt; a.out = out; a.out_f32 = out_dtype == SFG_F32;
    a.q_heads = static_cast<int>(q_heads); a.kv_heads = static_cast<int>(kv_heads);
    a.seq_q = static_cast<int>(seq_q); a.seq_kv = static_cast<int>(seq_kv);
    a.ld_vt = static_cast<int>(ld_vt); a.causal = causal;
    a.nqb = static_cast<int>((seq_q + bm - 1) / bm);
    a.scale_log2 = scale * kLog2e;
    a.xcds = device_xcds(stream);
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.nqb) * q_heads * batch));
    if (waves == 8) attn_prefill_fa2_kernel<8><<<grid, 512, 0, stream>>>(a);
    else attn_prefill_fa2_kernel<4><<<grid, 256, 0, stream>>>(a);
    return SFG_OK;
}

// ===========================================================================
// Paged Split-KV decode on MFMA, head_dim 128 or 64, 16-token pages.
//
// Pool layouts (one 4 KB run per (page, kv_head)):
//   K [page][Hkv][16 tokens][D dims]   V [page][Hkv][D dims][16 tokens]
// V is token-minor inside a page so that the MFMA operand V^T (dims x tokens)
// is read as 8-byte runs.  Per page a wave does
//   S^T[16 tok][16 q] = K[16 tok][D] Q^T[D][16 q]        D/32 x mfma_16x16x32_bf16
//   O^T[D][16 q] += V^T[D][16 tok] P^T[16 tok][16 q]      D/16 x mfma_16x16x16_bf16
// where the GQA group's G query heads occupy the first G columns.  In the
// S^T accumulator lane l holds query (l & 15) and tokens 4 (l >> 4) + r, which
// is exactly the P^T operand layout, and the O^T accumulator holds the same
// query per lane: the online softmax needs only a 4-lane max per page and a
// per-lane rescale.
// ===========================================================================
constexpr int kPageTok = 16;

typedef short short4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ short4v as_short4(const uint2& v) { return __builtin_bit_cast(short4v, v); }

template <int G, int kDecD>
__global__ __launch_bounds__(256) void attn_decode_split_kernel(
    const float* __restrict__ q, int64_t q_row_stride, const float* __restrict__ rope,
    int rope_pos, const uint16_t* __restrict__ k_pool, const uint16_t* __restrict__ v_pool,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ seq_lens, int uniform_len,
    int len_extra,
    int kv_heads, int pages_per_seq, int num_pages, int splits, float scale_log2,
    float* __restrict__ part_ml, float* __restrict__ part_acc) {
    static_assert(G >= 1 && G <= 16, "GQA group must fit the 16 MFMA columns");
    static_assert(kDecD == 64 || kDecD == 128, "head_dim 64 or 128");
    constexpr int kKs = kDecD / 32;   // k-steps of S^T = K Q^T
    constexpr int kDt = kDecD / 16;   // 16-dim blocks of O^T
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int q_heads = kv_heads * G;
    const int lr = lane & 15, lg = lane >> 4;
    // Tokens this sequence attends over: its length (plus len_extra tokens just
    // appended in place), at most the table's capacity; the query rotates at
    // rope_pos, or at the length before the append (its own position) when
    // rope_pos < 0 -- clamped to the capacity's last row, the last row a
    // capacity-sized RoPE table holds (a step past the capacity appended
    // nothing and is refused by the host mirror).
    const int capacity = pages_per_seq * kPageTok;
    const int len0 = seq_lens ? seq_lens[b] : uniform_len;
    const int len = min(len0 + len_extra, capacity);
    const int q_pos = rope_pos >= 0 ? rope_pos : min(max(len0, 0), capacity - 1);
    const int pages = (len + kPageTok - 1) / kPageTok;
    const int sp_begin = static_cast<int>(static_cast<int64_t>(pages) * split / splits);
    const int sp_end = static_cast<int>(static_cast<int64_t>(pages) * (split + 1) / splits);
    const int n_sp = sp_end - sp_begin;
    const int w_begin = sp_begin + n_sp * wave / 4;
    const int w_end = sp_begin + n_sp * (wave + 1) / 4;

    // Q^T operand: lane supplies query head lr (zero beyond the group), dims
    // 32 s + 8 lg + [0, 8), rotated by the host table at rope_pos when given.
    bf16x8 qf[kKs];
    {
        const bool has = lr < G;
        const float* qr = q + static_cast<int64_t>(b) * q_row_stride +
                          static_cast<int64_t>(kvh * G + (has ? lr : 0)) * kDecD;
        // every Q vector and rotation pair is loaded before the first use (one
        // memory round trip instead of one per k-step)
        float4 qa[kKs], qc[kKs];
        float2 rot[kKs][4];
#pragma unroll
        for (int s = 0; s < kKs; ++s) {
            qa[s] = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg);
            qc[s] = *reinterpret_cast<const float4*>(qr + 32 * s + 8 * lg + 4);
        }
        if (rope) {
            const float2* t = reinterpret_cast<const float2*>(rope) +
                              static_cast<int64_t>(q_pos) * (kDecD / 2) + 4 * lg;
#pragma unroll
            for (int s = 0; s < kKs; ++s)
#pragma unroll
                for (int e = 0; e < 4; ++e) rot[s][e] = t[16 * s + e];
        }
#pragma unroll
        for (int s = 0; s < kKs; ++s) {
            float v[8];
            const float4 a = qa[s];
            const float4 c = qc[s];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
            if (rope) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float2 cs = rot[s][e];
                    const float ev = v[2 * e], od = v[2 * e + 1];
                    v[2 * e] = ev * cs.x - od * cs.y;
                    v[2 * e + 1] = ev * cs.y + od * cs.x;
                }
            }
            if (!has) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = 0.f;
            }
            qf[s] = as_bf16x8(f32x8_to_bf16x8(v));
        }
    }

    floatx4 acc[kDt];
#pragma unroll
    for (int i = 0; i < kDt; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    const int32_t* ptab = page_table + static_cast<int64_t>(b) * pages_per_seq;
    const int64_t head_stride = static_cast<int64_t>(kPageTok) * kDecD;
    const int64_t page_stride = head_stride * kv_heads;
    // per-lane offsets inside a (page, kv_head) block
    const int k_off = lr * kDecD + 8 * lg;  // + 32 s
    const int v_off = lr * kPageTok + 4 * lg;  // + 16 dt * 16

    uint4 kb[kKs];
    uint2 vb[kDt];
    bool okb = false;
    // Long page ranges: the wave's page ids 64 at a time (lane i holds page
    // ids_base + i), so a page's K / V loads wait on no page-table read of
    // their own.  Short ranges read each id through the scalar cache, which
    // costs less than the one vector load up front.
    const bool vec_ids = w_end - w_begin > 16;
    int ids_vec = 0, ids_base = w_begin - 64;
    auto phys_of = [&](int pg) {
        if (!vec_ids) return ptab[pg];
        if (pg - ids_base >= 64) {  // wave-uniform
            ids_base = pg;
            ids_vec = pg + lane < w_end ? ptab[pg + lane] : -1;
        }
        return __builtin_amdgcn_readlane(ids_vec, pg - ids_base);
    };
    // Load page p (guarded: an id outside the pool reads nothing).
#define SFG_LOAD_PAGE(p)                                                                   \
    {                                                                                      \
        const int phys = phys_of(p);                                                       \
        okb = phys >= 0 && phys < num_pages;                                               \
        const int64_t base = okb ? static_cast<int64_t>(phys) * page_stride + kvh * head_stride : 0; \
        const uint16_t* kp = k_pool + base + k_off;                                        \
        const uint16_t* vp = v_pool + base + v_off;                                        \
        _Pragma("unroll") for (int s = 0; s < kKs; ++s)                                    \
            kb[s] = okb ? *reinterpret_cast<const uint4*>(kp + 32 * s) : make_uint4(0, 0, 0, 0); \
        _Pragma("unroll") for (int dt = 0; dt < kDt; ++dt)                                 \
            vb[dt] = okb ? *reinterpret_cast<const uint2*>(vp + dt * 16 * kPageTok) : make_uint2(0, 0); \
    }
    if (w_begin < w_end) SFG_LOAD_PAGE(w_begin);
    for (int p = w_begin; p < w_end; ++p) {
        uint4 kc[kKs];
        uint2 vc[kDt];
#pragma unroll
        for (int s = 0; s < kKs; ++s) kc[s] = kb[s];
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt) vc[dt] = vb[dt];
        const bool ok = okb;
        if (p + 1 < w_end) SFG_LOAD_PAGE(p + 1);
        floatx4 st = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kKs; ++s)
            st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kc[s]), qf[s], st, 0, 0, 0);
        // st[r]: token 16 p + 4 lg + r, query lr
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = p * kPageTok + 4 * lg + r;
            sv[r] = (ok && tok < len) ? st[r] * scale_log2 : -INFINITY;
            mx = fmaxf(mx, sv[r]);
        }
        mx = xor16_max(mx);
        mx = xor32_max(mx);
        const float m_new = fmaxf(m_run, mx);
        if (m_new != -INFINITY) {
            const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
            float pv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) pv[r] = (sv[r] == -INFINITY) ? 0.f : fast_exp2(sv[r] - m_new);
            l_run = l_run * alpha + (pv[0] + pv[1] + pv[2] + pv[3]);
            uint2 pk;
            pk.x = pack_bf16x2(pv[0], pv[1]);
            pk.y = pack_bf16x2(pv[2], pv[3]);
            const short4v pb = as_short4(pk);
#pragma unroll
            for (int dt = 0; dt < kDt; ++dt) {
                acc[dt] *= alpha;
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(as_short4(vc[dt]), pb, acc[dt], 0, 0, 0);
            }
            m_run = m_new;
        }
    }
#undef SFG_LOAD_PAGE
    l_run = xor16_sum(l_run);
    l_run = xor32_sum(l_run);

    // Merge the 4 waves in LDS.  acc[dt][r] = O^T[d = 16 dt + 4 lg + r][query lr].
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_acc[4][G][kDecD];
    if (lr < G) {
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) s_acc[wave][lr][16 * dt + 4 * lg + r] = acc[dt][r];
        if (lg == 0) {
            s_m[wave][lr] = m_run;
            s_l[wave][lr] = l_run;
        }
    }
    __syncthreads();
    for (int o = threadIdx.x; o < G * kDecD; o += 256) {
        const int g = o / kDecD, d = o % kDecD;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) mm = fmaxf(mm, s_m[w][g]);
        float ls = 0.f, as = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float wf = (s_m[w][g] == -INFINITY) ? 0.f : fast_exp2(s_m[w][g] - mm);
            ls += s_l[w][g] * wf;
            as += s_acc[w][g][d] * wf;
        }
        const int h = kvh * G + g;
        const int64_t slot = (static_cast<int64_t>(b) * q_heads + h) * splits + split;
        part_acc[slot * kDecD + d] = as;
        if (d == 0) {
            part_ml[slot * 2] = mm;
            part_ml[slot * 2 + 1] = ls;
        }
    }
}

// NS > 0: at most NS splits, merged from registers; NS = 0: any count.
template <typename OutT, int kDecD, int NS>
__global__ __launch_bounds__(kDecD) void attn_decode_combine_kernel(
    const float* __restrict__ part_ml, const float* __restrict__ part_acc, OutT* __restrict__ out,
    int splits) {
    const int bh = blockIdx.x;  // b * q_heads + h
    const int d = threadIdx.x;
    const float* ml = part_ml + static_cast<int64_t>(bh) * splits * 2;
    const float* pa = part_acc + static_cast<int64_t>(bh) * splits * kDecD + d;
    float mm = -INFINITY;
    float ls = 0.f, as = 0.f;
    if constexpr (NS > 0) {
        // every split's (m, l, acc) loaded before the merge: one memory wait.
        // Slots past the split count re-read the last split (no branch around
        // a load: a conditional load is waited for before the branches join)
        // and are left out of the sums.
        float m_s[NS], l_s[NS], a_s[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int sc = s < splits ? s : splits - 1;
            m_s[s] = ml[2 * sc];
            l_s[s] = ml[2 * sc + 1];
            a_s[s] = pa[sc * kDecD];
        }
        // the merge below branches on the (uniform) split maxima; an empty use
        // keeps the compiler from sinking the acc loads into those branches,
        // where they would be issued and waited for one at a time
#pragma unroll
        for (int s = 0; s < NS; ++s) asm volatile("" ::"v"(a_s[s]));
#pragma unroll
        for (int s = 0; s < NS; ++s)
            if (s < splits) mm = fmaxf(mm, m_s[s]);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if (s < splits) {
                const float wf = (m_s[s] == -INFINITY) ? 0.f : fast_exp2(m_s[s] - mm);
                ls += l_s[s] * wf;
                as += a_s[s] * wf;
            }
        }
    } else {
        for (int s = 0; s < splits; ++s) mm = fmaxf(mm, ml[2 * s]);
        for (int s = 0; s < splits; ++s) {
            const float ms = ml[2 * s];
            const float wf = (ms == -INFINITY) ? 0.f : fast_exp2(ms - mm);
            ls += ml[2 * s + 1] * wf;
            as += pa[s * kDecD] * wf;
        }
    }
    const float o = as / ls;
    // merged layout [B][Hq * D] == [b][h * D + d]
    if constexpr (sizeof(OutT) == 4) out[static_cast<int64_t>(bh) * kDecD + d] = o;
    else out[static_cast<int64_t>(bh) * kDecD + d] = f32_to_bf16(o);
}

int decode_split_count(int64_t batch, int64_t kv_heads, int64_t max_context, int64_t page_tokens,
                       int32_t requested) {
    const int64_t pages = (max_context + page_tokens - 1) / page_tokens;
    if (requested > 0) return static_cast<int>(requested < pages ? requested : (pages > 0 ? pages : 1));
    // Aim for >= 1024 workgroups while keeping >= 32 pages (8 per wave) each.
    int s = 1;
    while (batch * kv_heads * s < 1024 && pages / (s * 2) >= 32) s *= 2;
    return s;
}

size_t decode_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim, int splits) {
    const size_t slots = static_cast<size_t>(batch) * q_heads * splits;
    const size_t ml = ((slots * 2 * sizeof(float) + 255) / 256) * 256;
    const size_t acc = ((slots * head_dim * sizeof(float) + 255) / 256) * 256;
    return ml + acc;
}

bool decode_mfma_supported(int kv_dtype, int64_t head_dim, int64_t page_tokens, int64_t group,
                           int64_t seq_q) {
    return kv_dtype == SFG_BF16 && (head_dim == 128 || head_dim == 64) && page_tokens == kPageTok &&
           seq_q == 1 && (group == 1 || group == 2 || group == 4 || group == 8 || group == 16);
}

int launch_attn_decode_paged(const float* q, int64_t q_row_stride, const float* rope, int rope_pos,
                             const uint16_t* k_pool, const uint16_t* v_pool,
                             const int32_t* page_table, const int32_t* seq_lens, int64_t max_context,
                             int len_extra, void* out, int out_dtype, int64_t batch, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, int64_t page_tokens,
                             int64_t pages_per_seq, int64_t num_pages, int splits, float scale,
                             void* workspace, hipStream_t stream, hipEvent_t mid_event) {
    if ((head_dim != 128 && head_dim != 64) || page_tokens != kPageTok) return SFG_ERR_UNSUPPORTED;
    if (splits < 1) return SFG_ERR_SHAPE;
    const int group = static_cast<int>(q_heads / kv_heads);
    const size_t slots = static_cast<size_t>(batch) * q_heads * splits;
    float* part_ml = static_cast<float*>(workspace);
    float* part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                               ((slots * 2 * sizeof(float) + 255) / 256) * 256);
    const float scale_log2 = scale * kLog2e;
    const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(kv_heads),
                    static_cast<unsigned>(batch));
    const int len = static_cast<int>(max_context);
    const int pps = static_cast<int>(pages_per_seq);
    const int np = static_cast<int>(num_pages);
#define SFG_DECODE(G, D) attn_decode_split_kernel<G, D><<<grid, 256, 0, stream>>>(q, q_row_stride, rope, rope_pos, k_pool, v_pool, page_table, seq_lens, len, len_extra, static_cast<int>(kv_heads), pps, np, splits, scale_log2, part_ml, part_acc)
#define SFG_DECODE_G(D)                      \
    switch (group) {                         \
        case 1: SFG_DECODE(1, D); break;     \
        case 2: SFG_DECODE(2, D); break;     \
        case 4: SFG_DECODE(4, D); break;     \
        case 8: SFG_DECODE(8, D); break;     \
        case 16: SFG_DECODE(16, D); break;   \
        default: return SFG_ERR_UNSUPPORTED; \
    }
    if (head_dim == 128) {
        SFG_DECODE_G(128)
    } else {
        SFG_DECODE_G(64)
    }
#undef SFG_DECODE_G
#undef SFG_DECODE
    if (mid_event) (void)hipEventRecord(mid_event, stream);
    const dim3 cgrid(static_cast<unsigned>(batch * q_heads));
    auto combine = [&](auto* o, auto dcon) {
        using OutT = std::remove_pointer_t<decltype(o)>;
        constexpr int D = decltype(dcon)::value;
        if (splits <= 2) attn_decode_combine_kernel<OutT, D, 2><<<cgrid, D, 0, stream>>>(part_ml, part_acc, o, splits);
        else if (splits <= 4) attn_decode_combine_kernel<OutT, D, 4><<<cgrid, D, 0, stream>>>(part_ml, part_acc, o, splits);
        else if (splits <= 8) attn_decode_combine_kernel<OutT, D, 8><<<cgrid, D, 0, stream>>>(part_ml, part_acc, o, splits);
        else if (splits <= 16) attn_decode_combine_kernel<OutT, D, 16><<<cgrid, D, 0, stream>>>(part_ml, part_acc, o, splits);
        else attn_decode_combine_kernel<OutT, D, 0><<<cgrid, D, 0, stream>>>(part_ml, part_acc, o, splits);
    };
    if (head_dim == 128) {
        if (out_dtype == SFG_F32) combine(static_cast<float*>(out), std::integral_constant<int, 128>{});
        else combine(static_cast<uint16_t*>(out), std::integral_constant<int, 128>{});
    } else {
        if (out_dtype == SFG_F32) combine(static_cast<float*>(out), std::integral_constant<int, 64>{});
        else combine(static_cast<uint16_t*>(out), std::integral_constant<int, 64>{});
    }
    return SFG_OK;
}

// ===========================================================================
// Generic paged attention: any head_dim up to kRowMaxD, any page size, seq_q
// >= 1 new query rows per sequence under the causal offset j <= len - seq_q +
// i (attention_compiler.cpp:68-72), fp32 or bf16 pools; the decode path for
// the shapes the MFMA split kernel does not lower (fp32 caches, head dims
// other than 64 / 128, pages other than 16 tokens, more than one new token,
// GQA groups above 16).  One wave per (sequence, query row, query head,
// split): lane j scores key j of each 64-key chunk against the query held in
// LDS (one sequential fp32 FMA chain over the head dimension), then the wave
// accumulates p V with lane d owning dims d, d + 64, ... (online softmax,
// attention_compiler.cpp:102-112).  With more than one split each wave leaves
// its (m, l, acc) partial and attn_combine_rows_kernel merges them
// (merge_online, attention_compiler.cpp:132-145).  Q and the output are
// addressed by (batch, row, head) element strides: head-major [B][Hq][Sq][D]
// (the reference's attention layout) or merged rows [B][Sq][Hq][D]
// (merge_attention's, decoder_compiler.cpp:150-174).
// ===========================================================================
struct RowStrides {
    int64_t b, i, h;  // element strides of batch, query row and head; dims contiguous
    __device__ int64_t at(int bb, int ii, int hh) const {
        return bb * b + ii * i + static_cast<int64_t>(hh) * h;
    }
};

struct PagedRowsArgs {
    const float* q; RowStrides qs;
    const float2* rope; int rope_rows;      // optional [rope_rows][D/2] (cos, sin)
    int rope_pos;                           // >= 0: row i rotates at rope_pos + i; < 0: at seq_lens[b] + i
    const void* k_pool; const void* v_pool; // K [page][Hkv][pt][D], V [page][Hkv][D][pt]
    const int32_t* page_table; const int32_t* seq_lens;
    int uniform_len, len_extra;             // keys: (seq_lens ? seq_lens[b] : uniform_len) + len_extra
    void* out; int out_f32; RowStrides os;
    float* part_ml; float* part_acc;
    int q_heads, kv_heads, seq_q, head_dim, page_tokens, pages_per_seq, num_pages, splits, causal;
    float scale;
};

template <typename KvT>
__device__ __forceinline__ float kv_f32(const KvT* p, int64_t i) {
    if constexpr (sizeof(KvT) == 4) return p[i];
    else return bf16_to_f32(p[i]);
}

template <typename KvT>
__global__ __launch_bounds__(64) void attn_paged_rows_kernel(PagedRowsArgs p) {
    const int lane = threadIdx.x;
    const int slot = blockIdx.x;  // (b seq_q + i) q_heads + h
    const int split = blockIdx.y;
    const int h = slot % p.q_heads;
    const int bi = slot / p.q_heads;
    const int i = bi % p.seq_q, b = bi / p.seq_q;
    const int kvh = h * p.kv_heads / p.q_heads;
    const int D = p.head_dim, pt = p.page_tokens;
    const int capacity = p.pages_per_seq * pt;
    const int len0 = p.seq_lens ? p.seq_lens[b] : p.uniform_len;
    const int len = min(len0 + p.len_extra, capacity);
    const int kend = max(p.causal ? min(len, len - p.seq_q + i + 1) : len, 0);
    const int k0 = static_cast<int>(static_cast<int64_t>(kend) * split / p.splits);
    const int k1 = static_cast<int>(static_cast<int64_t>(kend) * (split + 1) / p.splits);

    __shared__ float sq[kRowMaxD];
    const float* qr = p.q + p.qs.at(b, i, h);
    for (int d = lane; d < D; d += 64) sq[d] = qr[d];
    __syncthreads();
    if (p.rope && p.rope_rows > 0) {
        const int pos = min(max((p.rope_pos >= 0 ? p.rope_pos : len0) + i, 0), p.rope_rows - 1);
        for (int t = lane; t < D / 2; t += 64) {
            const float2 cs = p.rope[static_cast<int64_t>(pos) * (D / 2) + t];
            const float e = sq[2 * t], o = sq[2 * t + 1];
            sq[2 * t] = e * cs.x - o * cs.y;
            sq[2 * t + 1] = e * cs.y + o * cs.x;
        }
        __syncthreads();
    }
    const KvT* kpool = static_cast<const KvT*>(p.k_pool);
    const KvT* vpool = static_cast<const KvT*>(p.v_pool);
    const int32_t* table = p.page_table + static_cast<int64_t>(b) * p.pages_per_seq;
    float m = -INFINITY, l = 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int base = k0; base < k1; base += 64) {
        const int j = base + lane;
        float s = -INFINITY;
        int page = -1;
        if (j < k1) {
            const int id = table[j / pt];
            if (id >= 0 && id < p.num_pages) {
                page = id;
                const KvT* kr = kpool + ((static_cast<int64_t>(id) * p.kv_heads + kvh) * pt + j % pt) * D;
                float dot = 0.f;
                for (int d = 0; d < D; ++d) dot = fmaf(sq[d], kv_f32(kr, d), dot);
                s = dot * p.scale;
            }
        }
        const float m_new = fmaxf(m, wave_max(s));
        if (m_new == -INFINITY) continue;  // wave-uniform: nothing visible in this chunk yet
        const float alpha = m == -INFINITY ? 0.f : expf(m - m_new);
        const float pr = s == -INFINITY ? 0.f : expf(s - m_new);
        l = l * alpha + wave_sum(pr);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= alpha;
        const int count = min(64, k1 - base);
        for (int t = 0; t < count; ++t) {
            const float pt_t = lane_bcast(pr, t);
            const int pg = lane_bcast(page, t);
            if (pg < 0) continue;  // wave-uniform
            const int jt = base + t;
            const KvT* vb = vpool + (static_cast<int64_t>(pg) * p.kv_heads + kvh) * D * pt + jt % pt;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = lane + 64 * r;
                if (d < D) acc[r] = fmaf(pt_t, kv_f32(vb, static_cast<int64_t>(d) * pt), acc[r]);
            }
        }
        m = m_new;
    }
    if (p.splits == 1) {
        const int64_t o0 = p.os.at(b, i, h);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = lane + 64 * r;
            if (d >= D) continue;
            const float o = acc[r] / l;  // no visible key: 0 / 0, as the reference's softmax gives
            if (p.out_f32) static_cast<float*>(p.out)[o0 + d] = o;
            else static_cast<uint16_t*>(p.out)[o0 + d] = f32_to_bf16(o);
        }
        return;
    }
    const int64_t part = static_cast<int64_t>(slot) * p.splits + split;
    if (lane == 0) {
        p.part_ml[2 * part] = m;
        p.part_ml[2 * part + 1] = l;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int d = lane + 64 * r;
        if (d < D) p.part_acc[part * D + d] = acc[r];
    }
}

// merge_online over a row's splits: weights e^(m_s - M), output sum / L.
__global__ __launch_bounds__(64) void attn_combine_rows_kernel(const float* __restrict__ part_ml,
                                                              const float* __restrict__ part_acc,
                                                              void* out, int out_f32, RowStrides os,
                                                              int q_heads, int seq_q, int head_dim,
                                                              int splits) {
    const int lane = threadIdx.x;
    const int64_t slot = blockIdx.x;  // (b seq_q + i) q_heads + h
    const int h = static_cast<int>(slot % q_heads);
    const int bi = static_cast<int>(slot / q_heads);
    const int64_t o0 = os.at(bi / seq_q, bi % seq_q, h);
    const int D = head_dim;
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s) M = fmaxf(M, part_ml[2 * (slot * splits + s)]);
    float L = 0.f;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < splits; ++s) {
        const int64_t part = slot * splits + s;
        const float ms = part_ml[2 * part];
        if (ms == -INFINITY) continue;
        const float w = expf(ms - M);
        L = fmaf(part_ml[2 * part + 1], w, L);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = lane + 64 * r;
            if (d < D) o[r] = fmaf(w, part_acc[part * D + d], o[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int d = lane + 64 * r;
        if (d >= D) continue;
        const float v = o[r] / L;
        if (out_f32) static_cast<float*>(out)[o0 + d] = v;
        else static_cast<uint16_t*>(out)[o0 + d] = f32_to_bf16(v);
    }
}

int paged_rows_split_count(int64_t rows, int64_t max_keys, int32_t requested) {
    if (requested > 0) return static_cast<int>(requested < max_keys ? requested : (max_keys > 0 ? max_keys : 1));
    // >= 1024 waves while every split keeps >= 256 keys
    int s = 1;
    while (rows * s < 1024 && max_keys / (s * 2) >= 256) s *= 2;
    return s;
}

size_t paged_rows_workspace_bytes(int64_t rows, int64_t head_dim, int splits) {
    if (splits <= 1) return 0;
    const size_t parts = static_cast<size_t>(rows) * splits;
    return ((parts * 2 * sizeof(float) + 255) / 256) * 256 + ((parts * head_dim * sizeof(float) + 255) / 256) * 256;
}

int launch_attn_paged_rows(const PagedRowsLaunch& a, void* workspace, hipStream_t stream) {
    if (a.head_dim < 1 || a.head_dim > kRowMaxD || a.page_tokens < 1 || a.splits < 1 || a.seq_q < 1)
        return SFG_ERR_UNSUPPORTED;
    if (a.kv_dtype != SFG_F32 && a.kv_dtype != SFG_BF16) return SFG_ERR_UNSUPPORTED;
    PagedRowsArgs p{};
    p.q = a.q; p.qs = RowStrides{a.q_stride_b, a.q_stride_i, a.q_stride_h};
    p.os = RowStrides{a.out_stride_b, a.out_stride_i, a.out_stride_h};
    p.rope = reinterpret_cast<const float2*>(a.rope); p.rope_rows = a.rope_rows; p.rope_pos = a.rope_pos;
    p.k_pool = a.k_pool; p.v_pool = a.v_pool;
    p.page_table = a.page_table; p.seq_lens = a.seq_lens;
    p.uniform_len = static_cast<int>(a.max_context); p.len_extra = a.len_extra;
    p.out = a.out; p.out_f32 = a.out_dtype == SFG_F32;
    const int64_t rows = a.batch * a.seq_q * a.q_heads;
    if (a.splits > 1) {
        const size_t parts = static_cast<size_t>(rows) * a.splits;
        p.part_ml = static_cast<float*>(workspace);
        p.part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                              ((parts * 2 * sizeof(float) + 255) / 256) * 256);
    }
    p.q_heads = static_cast<int>(a.q_heads); p.kv_heads = static_cast<int>(a.kv_heads);
    p.seq_q = static_cast<int>(a.seq_q); p.head_dim = static_cast<int>(a.head_dim);
    p.page_tokens = static_cast<int>(a.page_tokens); p.pages_per_seq = static_cast<int>(a.pages_per_seq);
    p.num_pages = static_cast<int>(a.num_pages); p.splits = a.splits; p.causal = a.causal;
    p.scale = a.scale;
    const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(a.splits));
    if (a.kv_dtype == SFG_F32) attn_paged_rows_kernel<float><<<grid, 64, 0, stream>>>(p);
    else attn_paged_rows_kernel<uint16_t><<<grid, 64, 0, stream>>>(p);
    if (a.mid_event) (void)hipEventRecord(a.mid_event, stream);
    if (a.splits > 1)
        attn_combine_rows_kernel<<<dim3(static_cast<unsigned>(rows)), 64, 0, stream>>>(
            p.part_ml, p.part_acc, a.out, p.out_f32, p.os, p.q_heads, p.seq_q, p.head_dim, a.splits);
    return SFG_OK;
}

// ===========================================================================
// Paged KV cache maintenance: append_paged_kv / gather_paged_kv
// (next_milestones.cpp:486-524, 554-581) on the device pools
// K [page][Hkv][page_tokens][D], V [page][Hkv][D][page_tokens] (fp32 or bf16)
// through per-sequence page tables [B][pages_per_seq].  Pages are assigned by
// the host (the plan's allocator, as the reference's free list); the kernels
// only move data and skip any position past the table's capacity or any page
// id outside the pool.  Any head_dim, any page size.
// ===========================================================================
struct KvAppendArgs {
    const void* keys; const void* values; int src_f32;
    int64_t sb, sh, st;           // source element strides: batch, kv head, token (dims contiguous)
    const float2* rope;           // [positions][D/2] (cos, sin) or null: keys rotated at their position
    void* k_pool; void* v_pool;
    const int32_t* page_table; const int32_t* seq_lens; int start;
    int kv_heads, head_dim, page_tokens, pages_per_seq, num_pages;
};

__device__ __forceinline__ float load_src(const void* base, int f32, int64_t idx) {
    if (f32) return static_cast<const float*>(base)[idx];
    return bf16_to_f32(static_cast<const uint16_t*>(base)[idx]);
}

template <typename KvT>
__device__ __forceinline__ KvT to_pool(float v) {
    if constexpr (sizeof(KvT) == 4) return v;
    else return f32_to_bf16(v);
}

// One wave per (token, kv_head, sequence); lane d owns dims d, d + 64, ...
// (with RoPE: pairs (2t, 2t + 1) for t = lane, lane + 64, ...).
template <typename KvT>
__global__ __launch_bounds__(64) void kv_append_kernel(KvAppendArgs a) {
    const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    const int D = a.head_dim, pt = a.page_tokens;
    const int pos = (a.seq_lens ? a.seq_lens[b] : a.start) + t;
    if (pos < 0 || pos >= a.pages_per_seq * pt) return;
    const int phys = a.page_table[static_cast<int64_t>(b) * a.pages_per_seq + pos / pt];
    if (phys < 0 || phys >= a.num_pages) return;
    const int slot = pos % pt;
    const int64_t src = b * a.sb + h * a.sh + t * a.st;
    const int64_t blk = static_cast<int64_t>(phys) * a.kv_heads + h;
    KvT* kdst = static_cast<KvT*>(a.k_pool) + (blk * pt + slot) * D;
    KvT* vdst = static_cast<KvT*>(a.v_pool) + blk * D * pt + slot;
    if (a.rope) {
        for (int q = lane; q < D / 2; q += 64) {
            const float e = load_src(a.keys, a.src_f32, src + 2 * q);
            const float o = load_src(a.keys, a.src_f32, src + 2 * q + 1);
            const float2 cs = a.rope[static_cast<int64_t>(pos) * (D / 2) + q];
            kdst[2 * q] = to_pool<KvT>(e * cs.x - o * cs.y);
            kdst[2 * q + 1] = to_pool<KvT>(e * cs.y + o * cs.x);
        }
        // an odd head_dim's last dimension is not rotated (apply_rope stops at d + 1 < D)
        if ((D & 1) && lane == 0) kdst[D - 1] = to_pool<KvT>(load_src(a.keys, a.src_f32, src + D - 1));
    } else {
        for (int d = lane; d < D; d += 64) kdst[d] = to_pool<KvT>(load_src(a.keys, a.src_f32, src + d));
    }
    for (int d = lane; d < D; d += 64)
        vdst[static_cast<int64_t>(d) * pt] = to_pool<KvT>(load_src(a.values, a.src_f32, src + d));
}

// Lengths advance by the appended tokens and saturate at the capacity: tokens
// past it were not written (kv_append_kernel skips them), so they are not
// counted either.
__global__ __launch_bounds__(256) void kv_advance_kernel(int32_t* seq_lens, int batch, int tokens,
                                                         int capacity) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b < batch) seq_lens[b] = min(seq_lens[b] + tokens, capacity);
}

// gather_paged_kv: pools -> keys / values [B][Hkv][length][D] fp32 (bf16 widened exactly).
template <typename KvT>
__global__ __launch_bounds__(64) void kv_gather_kernel(const KvT* __restrict__ k_pool,
                                                       const KvT* __restrict__ v_pool,
                                                       const int32_t* __restrict__ page_table,
                                                       int kv_heads, int head_dim, int page_tokens,
                                                       int pages_per_seq, int num_pages, int length,
                                                       float* __restrict__ keys,
                                                       float* __restrict__ values) {
    const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    const int D = head_dim, pt = page_tokens;
    const int phys = page_table[static_cast<int64_t>(b) * pages_per_seq + t / pt];
    const bool ok = phys >= 0 && phys < num_pages;
    const int slot = t % pt;
    const int64_t blk = static_cast<int64_t>(ok ? phys : 0) * kv_heads + h;
    const int64_t dst = ((static_cast<int64_t>(b) * kv_heads + h) * length + t) * D;
    for (int d = lane; d < D; d += 64) {
        keys[dst + d] = ok ? kv_f32(k_pool, (blk * pt + slot) * D + d) : 0.f;
        values[dst + d] = ok ? kv_f32(v_pool, (blk * D + d) * pt + slot) : 0.f;
    }
}

int launch_kv_append(const void* keys, const void* values, int src_dtype, int64_t sb, int64_t sh,
                     int64_t st, const float* rope, void* k_pool, void* v_pool, int pool_dtype,
                     const int32_t* page_table, int32_t* seq_lens, int64_t start, int advance,
                     int64_t batch, int64_t kv_heads, int64_t tokens, int64_t head_dim,
                     int64_t page_tokens, int64_t pages_per_seq, int64_t num_pages,
                     hipStream_t stream) {
    if (head_dim < 1 || page_tokens < 1) return SFG_ERR_UNSUPPORTED;
    if (pool_dtype != SFG_F32 && pool_dtype != SFG_BF16) return SFG_ERR_UNSUPPORTED;
    KvAppendArgs a{};
    a.keys = keys; a.values = values; a.src_f32 = src_dtype == SFG_F32;
    a.sb = sb; a.sh = sh; a.st = st;
    a.rope = reinterpret_cast<const float2*>(rope);
    a.k_pool = k_pool; a.v_pool = v_pool; a.page_table = page_table; a.seq_lens = seq_lens;
    a.start = static_cast<int>(start);
    a.kv_heads = static_cast<int>(kv_heads); a.head_dim = static_cast<int>(head_dim);
    a.page_tokens = static_cast<int>(page_tokens); a.pages_per_seq = static_cast<int>(pages_per_seq);
    a.num_pages = static_cast<int>(num_pages);
    const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(kv_heads), static_cast<unsigned>(batch));
    if (pool_dtype == SFG_F32) kv_append_kernel<float><<<grid, 64, 0, stream>>>(a);
    else kv_append_kernel<uint16_t><<<grid, 64, 0, stream>>>(a);
    if (advance && seq_lens)
        kv_advance_kernel<<<dim3(static_cast<unsigned>((batch + 255) / 256)), 256, 0, stream>>>(
            seq_lens, static_cast<int>(batch), static_cast<int>(tokens),
            static_cast<int>(pages_per_seq * page_tokens));
    return SFG_OK;
}

void launch_kv_advance(int32_t* seq_lens, int64_t batch, int64_t tokens, int64_t capacity,
                       hipStream_t stream) {
    kv_advance_kernel<<<dim3(static_cast<unsigned>((batch + 255) / 256)), 256, 0, stream>>>(
        seq_lens, static_cast<int>(batch), static_cast<int>(tokens), static_cast<int>(capacity));
}

int launch_kv_gather(const void* k_pool, const void* v_pool, int pool_dtype, const int32_t* page_table,
                     int64_t batch, int64_t kv_heads, int64_t length, int64_t head_dim,
                     int64_t page_tokens, int64_t pages_per_seq, int64_t num_pages, float* keys,
                     float* values, hipStream_t stream) {
    if (head_dim < 1 || page_tokens < 1) return SFG_ERR_UNSUPPORTED;
    if (pool_dtype != SFG_F32 && pool_dtype != SFG_BF16) return SFG_ERR_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>(length), static_cast<unsigned>(kv_heads), static_cast<unsigned>(batch));
    const int kvh = static_cast<int>(kv_heads), d = static_cast<int>(head_dim), pt = static_cast<int>(page_tokens);
    const int pps = static_cast<int>(pages_per_seq), np = static_cast<int>(num_pages), len = static_cast<int>(length);
    if (pool_dtype == SFG_F32)
        kv_gather_kernel<float><<<grid, 64, 0, stream>>>(static_cast<const float*>(k_pool),
                                                         static_cast<const float*>(v_pool), page_table,
                                                         kvh, d, pt, pps, np, len, keys, values);
    else
        kv_gather_kernel<uint16_t><<<grid, 64, 0, stream>>>(static_cast<const uint16_t*>(k_pool),
                                                            static_cast<const uint16_t*>(v_pool), page_table,
                                                            kvh, d, pt, pps, np, len, keys, values);
    return SFG_OK;
}

}  // namespace sfg
