// sfg_attention.hip -- GQA attention for gfx950.
//
//  * attn_prefill_f32_kernel: fp32 online softmax (attention_compiler.cpp:286-377),
//    one wave per query row, 64 keys per step (one per lane), values
//    accumulated with the wave owning the head dimension.
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
//    once; lanes split a 16-token page as 4 tokens x 16 chunks of 8 dims, pages
//    are double-buffered in registers, waves merge in LDS, splits merge in a
//    second small kernel.
#include "sfg_kernels.hpp"

namespace sfg {

// ===========================================================================
// fp32 prefill
// ===========================================================================
template <typename OutT>
__global__ __launch_bounds__(256) void attn_prefill_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    OutT* __restrict__ out, int q_heads, int kv_heads, int seq_q, int seq_kv, int head_dim,
    int causal, float scale) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int qi = blockIdx.x * 4 + wave;
    const int h = blockIdx.y, b = blockIdx.z;
    __shared__ float sq[4][128];
    if (qi >= seq_q) return;
    const int kvh = h * kv_heads / q_heads;
    const float* qr = q + ((static_cast<int64_t>(b) * q_heads + h) * seq_q + qi) * head_dim;
    for (int d = lane; d < head_dim; d += 64) sq[wave][d] = qr[d];
    __builtin_amdgcn_wave_barrier();
    const float* kb = k + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * head_dim;
    const float* vb = v + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * head_dim;
    const int limit = causal ? (seq_kv - seq_q + qi) : (seq_kv - 1);
    float m = -INFINITY, l = 0.f;
    float acc0 = 0.f, acc1 = 0.f;  // dims lane, lane + 64
    for (int base = 0; base <= limit && base < seq_kv; base += 64) {
        const int j = base + lane;
        float s = -INFINITY;
        if (j <= limit && j < seq_kv) {
            const float* kr = kb + static_cast<int64_t>(j) * head_dim;
            float dot = 0.f;
            for (int d = 0; d < head_dim; ++d) dot = fmaf(sq[wave][d], kr[d], dot);
            s = dot * scale;
        }
        const float mx = wave_max(s);
        const float m_new = fmaxf(m, mx);
        const float alpha = (m == -INFINITY) ? 0.f : expf(m - m_new);
        const float p = (s == -INFINITY) ? 0.f : expf(s - m_new);
        l = l * alpha + wave_sum(p);
        acc0 *= alpha;
        acc1 *= alpha;
        const int count = min(64, min(limit, seq_kv - 1) - base + 1);
        for (int t = 0; t < count; ++t) {
            const float pt = __shfl(p, t, 64);
            const float* vr = vb + static_cast<int64_t>(base + t) * head_dim;
            if (lane < head_dim) acc0 = fmaf(pt, vr[lane], acc0);
            if (lane + 64 < head_dim) acc1 = fmaf(pt, vr[lane + 64], acc1);
        }
        m = m_new;
    }
    const int64_t row = static_cast<int64_t>(b) * seq_q + qi;
    OutT* orow = out + row * (static_cast<int64_t>(q_heads) * head_dim) + h * head_dim;
    if (lane < head_dim) {
        const float o = acc0 / l;
        if constexpr (sizeof(OutT) == 4) orow[lane] = o; else orow[lane] = f32_to_bf16(o);
    }
    if (lane + 64 < head_dim) {
        const float o = acc1 / l;
        if constexpr (sizeof(OutT) == 4) orow[lane + 64] = o; else orow[lane + 64] = f32_to_bf16(o);
    }
}

void launch_attn_prefill_f32(const float* q, const float* k, const float* v, void* out,
                             int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t seq_q, int64_t seq_kv, int64_t head_dim, int causal,
                             float scale, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((seq_q + 3) / 4), static_cast<unsigned>(q_heads),
                    static_cast<unsigned>(batch));
    if (out_dtype == SFG_F32)
        attn_prefill_f32_kernel<float><<<grid, 256, 0, stream>>>(
            q, k, v, static_cast<float*>(out), q_heads, kv_heads, seq_q, seq_kv, head_dim, causal,
            scale);
    else
        attn_prefill_f32_kernel<uint16_t><<<grid, 256, 0, stream>>>(
            q, k, v, static_cast<uint16_t*>(out), q_heads, kv_heads, seq_q, seq_kv, head_dim,
            causal, scale);
}

// ===========================================================================
// bf16 MFMA flash prefill, head_dim 128.
// ===========================================================================
constexpr int kFaD = 128;
constexpr int kFaBM = 128;          // query rows per workgroup
constexpr int kFaBN = 64;           // keys per tile
constexpr int kKRow = kFaD + 8;     // padded K row (bf16 elements)
constexpr int kVRow = kFaBN + 8;    // padded V^T row

template <typename OutT>
__global__ __launch_bounds__(256) void attn_prefill_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, OutT* __restrict__ out, int q_heads, int kv_heads,
    int seq_q, int seq_kv, int causal, float scale_log2) {
    __shared__ __attribute__((aligned(16))) uint16_t sK[kFaBN * kKRow];
    __shared__ __attribute__((aligned(16))) uint16_t sVt[kFaD * kVRow];

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
    bf16x8 qf[8];
    {
        const uint16_t* qr = q + ((static_cast<int64_t>(b) * q_heads + h) * seq_q + my_q) * kFaD;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            uint4 val = make_uint4(0, 0, 0, 0);
            if (my_q < seq_q) val = *reinterpret_cast<const uint4*>(qr + s * 16 + half * 8);
            qf[s] = as_bf16x8(val);
        }
    }
    const uint16_t* kb = k + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * kFaD;
    const uint16_t* vb = v + (static_cast<int64_t>(b) * kv_heads + kvh) * seq_kv * kFaD;

    floatx16 acc_o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
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
        // Stage K [64][128] and V^T [128][64]: 1024 16-byte chunks each.
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int idx = tid + it * 256;
            const int key = idx >> 4;
            const int chunk = (idx & 15) * 8;
            uint4 kv4 = make_uint4(0, 0, 0, 0), vv4 = make_uint4(0, 0, 0, 0);
            if (kv0 + key < seq_kv) {
                kv4 = *reinterpret_cast<const uint4*>(kb + static_cast<int64_t>(kv0 + key) * kFaD + chunk);
                vv4 = *reinterpret_cast<const uint4*>(vb + static_cast<int64_t>(kv0 + key) * kFaD + chunk);
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
            for (int s = 0; s < 8; ++s) {
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
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
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
        for (int i = 0; i < 4; ++i)
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
                for (int i = 0; i < 4; ++i) {
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
    OutT* orow = out + row * (static_cast<int64_t>(q_heads) * kFaD) + h * kFaD;
#pragma unroll
    for (int i = 0; i < 4; ++i)
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
    if (head_dim != kFaD) return SFG_ERR_UNSUPPORTED;
    const float scale_log2 = scale * kLog2e;
    const dim3 grid(static_cast<unsigned>((seq_q + kFaBM - 1) / kFaBM),
                    static_cast<unsigned>(q_heads), static_cast<unsigned>(batch));
    if (out_dtype == SFG_F32)
        attn_prefill_bf16_kernel<float><<<grid, 256, 0, stream>>>(
            q, k, v, static_cast<float*>(out), q_heads, kv_heads, seq_q, seq_kv, causal, scale_log2);
    else
        attn_prefill_bf16_kernel<uint16_t><<<grid, 256, 0, stream>>>(
            q, k, v, static_cast<uint16_t*>(out), q_heads, kv_heads, seq_q, seq_kv, causal,
            scale_log2);
    return SFG_OK;
}

// ===========================================================================
// Paged Split-KV decode, head_dim 128, 16-token pages.
// ===========================================================================
constexpr int kDecD = 128;
constexpr int kPageTok = 16;

template <int G>
__global__ __launch_bounds__(256) void attn_decode_split_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ page_table,
    const int32_t* __restrict__ seq_lens, int uniform_len, int kv_heads, int pages_per_seq,
    int num_pages, int splits, float scale_log2, float* __restrict__ part_ml,
    float* __restrict__ part_acc) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int q_heads = kv_heads * G;
    const int len = min(seq_lens ? seq_lens[b] : uniform_len, pages_per_seq * kPageTok);
    const int pages = (len + kPageTok - 1) / kPageTok;
    // Pages of this split, then of this wave (contiguous ranges).
    const int sp_begin = static_cast<int>(static_cast<int64_t>(pages) * split / splits);
    const int sp_end = static_cast<int>(static_cast<int64_t>(pages) * (split + 1) / splits);
    const int n_sp = sp_end - sp_begin;
    const int w_begin = sp_begin + n_sp * wave / 4;
    const int w_end = sp_begin + n_sp * (wave + 1) / 4;

    const int dc = (lane & 15) * 8;  // 8 dims per lane
    const int ts = lane >> 4;        // token slot 0..3 within each group of 4 tokens

    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qr = q + (static_cast<int64_t>(b) * q_heads + kvh * G + g) * kDecD + dc;
        const float4 a = *reinterpret_cast<const float4*>(qr);
        const float4 c = *reinterpret_cast<const float4*>(qr + 4);
        qv[g][0] = a.x * scale_log2; qv[g][1] = a.y * scale_log2;
        qv[g][2] = a.z * scale_log2; qv[g][3] = a.w * scale_log2;
        qv[g][4] = c.x * scale_log2; qv[g][5] = c.y * scale_log2;
        qv[g][6] = c.z * scale_log2; qv[g][7] = c.w * scale_log2;
    }
    float m_run[G], l_run[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    }

    const int32_t* ptab = page_table + static_cast<int64_t>(b) * pages_per_seq;
    const int64_t head_stride = static_cast<int64_t>(kPageTok) * kDecD;       // one (page, kv_head)
    const int64_t page_stride = head_stride * kv_heads;
    auto page_ptr = [&](int p, const uint16_t* pool) -> const uint16_t* {
        const int phys = ptab[p];
        return pool + static_cast<int64_t>(phys) * page_stride + kvh * head_stride +
               static_cast<int64_t>(ts) * kDecD + dc;
    };
    auto page_ok = [&](int p) -> bool {
        const int phys = ptab[p];
        return phys >= 0 && phys < num_pages;
    };

    uint4 kbuf[4], vbuf[4];
    auto load_page = [&](int p) {
        if (page_ok(p)) {
            const uint16_t* kp = page_ptr(p, k_pool);
            const uint16_t* vp = page_ptr(p, v_pool);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                kbuf[u] = *reinterpret_cast<const uint4*>(kp + u * 4 * kDecD);
                vbuf[u] = *reinterpret_cast<const uint4*>(vp + u * 4 * kDecD);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) { kbuf[u] = make_uint4(0, 0, 0, 0); vbuf[u] = kbuf[u]; }
        }
    };
    if (w_begin < w_end) load_page(w_begin);
    for (int p = w_begin; p < w_end; ++p) {
        uint4 kc[4], vc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) { kc[u] = kbuf[u]; vc[u] = vbuf[u]; }
        const bool ok = page_ok(p);
        if (p + 1 < w_end) load_page(p + 1);
        // scores s[u][g] for token 16 p + 4 u + ts
        float s[4][G];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float kf[8];
            const uint32_t* kw = reinterpret_cast<const uint32_t*>(&kc[u]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kf[2 * e] = __uint_as_float(kw[e] << 16);
                kf[2 * e + 1] = __uint_as_float(kw[e] & 0xFFFF0000u);
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qv[g][e], kf[e], d);
                s[u][g] = d;
            }
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1)
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int g = 0; g < G; ++g) s[u][g] += __shfl_xor(s[u][g], off, 64);
        float mx[G];
#pragma unroll
        for (int g = 0; g < G; ++g) mx[g] = -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int tok = p * kPageTok + 4 * u + ts;
            const bool valid = ok && tok < len;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                if (!valid) s[u][g] = -INFINITY;
                mx[g] = fmaxf(mx[g], s[u][g]);
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            mx[g] = fmaxf(mx[g], __shfl_xor(mx[g], 16, 64));
            mx[g] = fmaxf(mx[g], __shfl_xor(mx[g], 32, 64));
        }
        float vf[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t* vw = reinterpret_cast<const uint32_t*>(&vc[u]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vf[u][2 * e] = __uint_as_float(vw[e] << 16);
                vf[u][2 * e + 1] = __uint_as_float(vw[e] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float m_new = fmaxf(m_run[g], mx[g]);
            if (m_new == -INFINITY) continue;  // nothing valid yet (uniform across the wave)
            const float alpha = (m_run[g] == -INFINITY) ? 0.f : fast_exp2(m_run[g] - m_new);
            l_run[g] *= alpha;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float pu = (s[u][g] == -INFINITY) ? 0.f : fast_exp2(s[u][g] - m_new);
                l_run[g] += pu;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pu, vf[u][e], acc[g][e]);
            }
            m_run[g] = m_new;
        }
    }
    // Combine the 4 token slots of the wave (lanes l, l^16, l^32, l^48).
#pragma unroll
    for (int g = 0; g < G; ++g) {
        l_run[g] += __shfl_xor(l_run[g], 16, 64);
        l_run[g] += __shfl_xor(l_run[g], 32, 64);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            acc[g][e] += __shfl_xor(acc[g][e], 16, 64);
            acc[g][e] += __shfl_xor(acc[g][e], 32, 64);
        }
    }
    // Merge the 4 waves in LDS.
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_acc[4][G][kDecD];
    if (lane < 16) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) s_acc[wave][g][dc + e] = acc[g][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) { s_m[wave][g] = m_run[g]; s_l[wave][g] = l_run[g]; }
    }
    __syncthreads();
    // thread -> (g, d): G * 128 outputs over 256 threads
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

template <typename OutT>
__global__ __launch_bounds__(128) void attn_decode_combine_kernel(
    const float* __restrict__ part_ml, const float* __restrict__ part_acc, OutT* __restrict__ out,
    int q_heads, int splits) {
    const int bh = blockIdx.x;  // b * q_heads + h
    const int d = threadIdx.x;
    const float* ml = part_ml + static_cast<int64_t>(bh) * splits * 2;
    float mm = -INFINITY;
    for (int s = 0; s < splits; ++s) mm = fmaxf(mm, ml[2 * s]);
    float ls = 0.f, as = 0.f;
    for (int s = 0; s < splits; ++s) {
        const float ms = ml[2 * s];
        const float wf = (ms == -INFINITY) ? 0.f : fast_exp2(ms - mm);
        ls += ml[2 * s + 1] * wf;
        as += part_acc[(static_cast<int64_t>(bh) * splits + s) * kDecD + d] * wf;
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
    // Aim for >= 1024 workgroups with >= 8 pages per workgroup (2 per wave).
    int s = 1;
    while (batch * kv_heads * s < 1024 && pages / (s * 2) >= 8) s *= 2;
    return s;
}

size_t decode_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim, int splits) {
    const size_t slots = static_cast<size_t>(batch) * q_heads * splits;
    const size_t ml = ((slots * 2 * sizeof(float) + 255) / 256) * 256;
    const size_t acc = ((slots * head_dim * sizeof(float) + 255) / 256) * 256;
    return ml + acc;
}

int launch_attn_decode_paged(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                             const int32_t* page_table, const int32_t* seq_lens, int64_t max_context,
                             void* out, int out_dtype, int64_t batch, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, int64_t page_tokens,
                             int64_t pages_per_seq, int64_t num_pages, int splits, float scale,
                             void* workspace, hipStream_t stream, hipEvent_t mid_event) {
    if (head_dim != kDecD || page_tokens != kPageTok) return SFG_ERR_UNSUPPORTED;
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
    switch (group) {
        case 1: attn_decode_split_kernel<1><<<grid, 256, 0, stream>>>(q, k_pool, v_pool, page_table, seq_lens, len, kv_heads, pps, np, splits, scale_log2, part_ml, part_acc); break;
        case 2: attn_decode_split_kernel<2><<<grid, 256, 0, stream>>>(q, k_pool, v_pool, page_table, seq_lens, len, kv_heads, pps, np, splits, scale_log2, part_ml, part_acc); break;
        case 4: attn_decode_split_kernel<4><<<grid, 256, 0, stream>>>(q, k_pool, v_pool, page_table, seq_lens, len, kv_heads, pps, np, splits, scale_log2, part_ml, part_acc); break;
        case 8: attn_decode_split_kernel<8><<<grid, 256, 0, stream>>>(q, k_pool, v_pool, page_table, seq_lens, len, kv_heads, pps, np, splits, scale_log2, part_ml, part_acc); break;
        default: return SFG_ERR_UNSUPPORTED;
    }
    if (mid_event) (void)hipEventRecord(mid_event, stream);
    const dim3 cgrid(static_cast<unsigned>(batch * q_heads));
    if (out_dtype == SFG_F32)
        attn_decode_combine_kernel<float><<<cgrid, kDecD, 0, stream>>>(
            part_ml, part_acc, static_cast<float*>(out), static_cast<int>(q_heads), splits);
    else
        attn_decode_combine_kernel<uint16_t><<<cgrid, kDecD, 0, stream>>>(
            part_ml, part_acc, static_cast<uint16_t*>(out), static_cast<int>(q_heads), splits);
    return SFG_OK;
}

}  // namespace sfg
