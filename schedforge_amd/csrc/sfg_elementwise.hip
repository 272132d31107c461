// sfg_elementwise.hip -- HBM-bound row kernels: RMSNorm, split+RoPE, weight
// packing / quantisation, fp32->bf16.
//
// All of these move each byte once; launches are sized to put >= 2 workgroups
// per CU on the 256-CU part and every global access is 16-byte vectorised where
// the row width allows.
#include "sfg_kernels.hpp"

#include <type_traits>

namespace sfg {

// ---------------------------------------------------------------------------
// RMSNorm (decoder_compiler.cpp:41-62).  One workgroup per row; 256 threads
// stream the row with float4 loads, sum squares in double (the reference's
// accumulator type), reduce across the wave with shuffles and across waves in
// LDS, then scale.  inverse = 1/sqrtf(float(sum/width) + eps), both correctly
// rounded (hipcc's default for sqrtf and fp32 division).
// ---------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      OutT* __restrict__ y, int width, float eps,
                                                      float* __restrict__ y32) {
    const int row = blockIdx.x;
    const float* xr = x + static_cast<int64_t>(row) * width;
    OutT* yr = y + static_cast<int64_t>(row) * width;
    __shared__ double partial[4];
    __shared__ float inv_shared;
    double sum = 0.0;
    const bool vec = (width & 3) == 0;
    if (vec) {
        for (int c = threadIdx.x * 4; c < width; c += 256 * 4) {
            const float4 v = *reinterpret_cast<const float4*>(xr + c);
            sum += static_cast<double>(v.x) * v.x;
            sum += static_cast<double>(v.y) * v.y;
            sum += static_cast<double>(v.z) * v.z;
            sum += static_cast<double>(v.w) * v.w;
        }
    } else {
        for (int c = threadIdx.x; c < width; c += 256) sum += static_cast<double>(xr[c]) * xr[c];
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        const double total = partial[0] + partial[1] + partial[2] + partial[3];
        inv_shared = 1.0f / sqrtf(static_cast<float>(total / static_cast<double>(width)) + eps);
    }
    __syncthreads();
    const float inv = inv_shared;
    if (vec) {
        for (int c = threadIdx.x * 4; c < width; c += 256 * 4) {
            const float4 v = *reinterpret_cast<const float4*>(xr + c);
            const float4 g = *reinterpret_cast<const float4*>(w + c);
            const float o0 = v.x * inv * g.x, o1 = v.y * inv * g.y;
            const float o2 = v.z * inv * g.z, o3 = v.w * inv * g.w;
            if constexpr (sizeof(OutT) == 4) {
                *reinterpret_cast<float4*>(yr + c) = make_float4(o0, o1, o2, o3);
            } else {
                uint2 packed;
                packed.x = pack_bf16x2(o0, o1);
                packed.y = pack_bf16x2(o2, o3);
                *reinterpret_cast<uint2*>(yr + c) = packed;
            }
            if (y32) *reinterpret_cast<float4*>(y32 + static_cast<int64_t>(row) * width + c) = make_float4(o0, o1, o2, o3);
        }
    } else {
        for (int c = threadIdx.x; c < width; c += 256) {
            const float o = xr[c] * inv * w[c];
            if constexpr (sizeof(OutT) == 4) yr[c] = o;
            else yr[c] = f32_to_bf16(o);
            if (y32) y32[static_cast<int64_t>(row) * width + c] = o;
        }
    }
}

// Rows of at most 1024 * NV floats (width a multiple of 4): the row and the
// gains are read once into registers before the reduction, so the output pass
// waits on no second global read.  Same accumulation order as rmsnorm_kernel
// (thread-strided float4 runs, wave sums, four partials), so the same bits.
template <typename OutT, int NV>
__global__ __launch_bounds__(256) void rmsnorm_reg_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          OutT* __restrict__ y, int width, float eps,
                                                          float* __restrict__ y32) {
    const int row = blockIdx.x;
    const float* xr = x + static_cast<int64_t>(row) * width;
    OutT* yr = y + static_cast<int64_t>(row) * width;
    __shared__ double partial[4];
    __shared__ float inv_shared;
    float4 v[NV], g[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (threadIdx.x + 256 * i) * 4;
        v[i] = c < width ? *reinterpret_cast<const float4*>(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        g[i] = c < width ? *reinterpret_cast<const float4*>(w + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if ((static_cast<int>(threadIdx.x) + 256 * i) * 4 >= width) break;
        sum += static_cast<double>(v[i].x) * v[i].x;
        sum += static_cast<double>(v[i].y) * v[i].y;
        sum += static_cast<double>(v[i].z) * v[i].z;
        sum += static_cast<double>(v[i].w) * v[i].w;
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        const double total = partial[0] + partial[1] + partial[2] + partial[3];
        inv_shared = 1.0f / sqrtf(static_cast<float>(total / static_cast<double>(width)) + eps);
    }
    __syncthreads();
    const float inv = inv_shared;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (threadIdx.x + 256 * i) * 4;
        if (c >= width) break;
        const float o0 = v[i].x * inv * g[i].x, o1 = v[i].y * inv * g[i].y;
        const float o2 = v[i].z * inv * g[i].z, o3 = v[i].w * inv * g[i].w;
        if constexpr (sizeof(OutT) == 4) {
            *reinterpret_cast<float4*>(yr + c) = make_float4(o0, o1, o2, o3);
        } else {
            uint2 packed;
            packed.x = pack_bf16x2(o0, o1);
            packed.y = pack_bf16x2(o2, o3);
            *reinterpret_cast<uint2*>(yr + c) = packed;
        }
        if (y32) *reinterpret_cast<float4*>(y32 + static_cast<int64_t>(row) * width + c) = make_float4(o0, o1, o2, o3);
    }
}

void launch_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int64_t rows,
                    int64_t width, float eps, hipStream_t stream, float* y32) {
    if (width % 4 == 0 && width <= 1024 * 8) {
        const int nv = width <= 1024 * 2 ? 2 : (width <= 1024 * 4 ? 4 : 8);
        auto go = [&](auto* out) {
            using OutT = std::remove_pointer_t<decltype(out)>;
            if (nv == 2) rmsnorm_reg_kernel<OutT, 2><<<dim3(rows), dim3(256), 0, stream>>>(x, w, out, static_cast<int>(width), eps, y32);
            else if (nv == 4) rmsnorm_reg_kernel<OutT, 4><<<dim3(rows), dim3(256), 0, stream>>>(x, w, out, static_cast<int>(width), eps, y32);
            else rmsnorm_reg_kernel<OutT, 8><<<dim3(rows), dim3(256), 0, stream>>>(x, w, out, static_cast<int>(width), eps, y32);
        };
        if (y_dtype == SFG_F32) go(static_cast<float*>(y));
        else go(static_cast<uint16_t*>(y));
        return;
    }
    if (y_dtype == SFG_F32)
        rmsnorm_kernel<float><<<dim3(rows), dim3(256), 0, stream>>>(x, w, static_cast<float*>(y),
                                                                     static_cast<int>(width), eps, y32);
    else
        rmsnorm_kernel<uint16_t><<<dim3(rows), dim3(256), 0, stream>>>(
            x, w, static_cast<uint16_t*>(y), static_cast<int>(width), eps, y32);
}

// ---------------------------------------------------------------------------
// split_qkv + apply_rope (decoder_compiler.cpp:96-148).  One thread per
// (row, head-slot, unit): Q heads, then K heads, then V heads of one row; a
// unit is the pair (2u, 2u + 1), and for an odd head_dim the last dimension,
// which apply_rope leaves unrotated (its loop stops at dimension + 1 <
// head_dim).  The rotation uses the host-built table (cos, sin per position
// and pair), whose float expressions are the reference's, so no device libm
// enters the angle.
// ---------------------------------------------------------------------------
template <typename OutT>
__device__ __forceinline__ void store_act(OutT* dst, float v) {
    if constexpr (sizeof(OutT) == 4) *dst = v;
    else *dst = f32_to_bf16(v);
}

template <typename OutT>
__global__ __launch_bounds__(256) void split_rope_kernel(
    const float* __restrict__ qkv, const float2* __restrict__ table, int batch, int seq,
    int q_heads, int kv_heads, int head_dim, OutT* __restrict__ q, OutT* __restrict__ k,
    OutT* __restrict__ v) {
    const int half = head_dim >> 1;
    const int units = (head_dim + 1) >> 1;
    const int heads_total = q_heads + 2 * kv_heads;
    const int64_t total = static_cast<int64_t>(batch) * seq * heads_total * units;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int unit = static_cast<int>(idx % units);
    const int64_t rest = idx / units;
    const int slot = static_cast<int>(rest % heads_total);
    const int64_t row = rest / heads_total;
    const int b = static_cast<int>(row / seq);
    const int s = static_cast<int>(row % seq);
    const int64_t width = static_cast<int64_t>(heads_total) * head_dim;
    const float* src = qkv + row * width + static_cast<int64_t>(slot) * head_dim + 2 * unit;
    OutT* dst;
    if (slot < q_heads) {
        dst = q + ((static_cast<int64_t>(b) * q_heads + slot) * seq + s) * head_dim;
    } else if (slot < q_heads + kv_heads) {
        if (k == nullptr) return;
        dst = k + ((static_cast<int64_t>(b) * kv_heads + (slot - q_heads)) * seq + s) * head_dim;
    } else {
        if (v == nullptr) return;
        dst = v + ((static_cast<int64_t>(b) * kv_heads + (slot - q_heads - kv_heads)) * seq + s) *
                      head_dim;
    }
    dst += 2 * unit;
    if (unit == half) {  // odd head_dim: the last dimension is copied as is
        store_act(dst, src[0]);
        return;
    }
    const float e = src[0], o = src[1];
    float o0 = e, o1 = o;
    if (slot < q_heads + kv_heads) {
        const float2 cs = table[static_cast<int64_t>(s) * half + unit];
        o0 = e * cs.x - o * cs.y;
        o1 = e * cs.y + o * cs.x;
    }
    store_act(dst, o0);
    store_act(dst + 1, o1);
}

void launch_split_rope(const float* qkv, const float* table, int64_t batch, int64_t seq,
                       int64_t q_heads, int64_t kv_heads, int64_t head_dim, void* q, void* k,
                       void* v, int out_dtype, hipStream_t stream) {
    const int64_t total = batch * seq * (q_heads + 2 * kv_heads) * ((head_dim + 1) / 2);
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    const float2* t = reinterpret_cast<const float2*>(table);
    if (out_dtype == SFG_F32)
        split_rope_kernel<float><<<grid, 256, 0, stream>>>(
            qkv, t, batch, seq, q_heads, kv_heads, head_dim, static_cast<float*>(q),
            static_cast<float*>(k), static_cast<float*>(v));
    else
        split_rope_kernel<uint16_t><<<grid, 256, 0, stream>>>(
            qkv, t, batch, seq, q_heads, kv_heads, head_dim, static_cast<uint16_t*>(q),
            static_cast<uint16_t*>(k), static_cast<uint16_t*>(v));
}

// ---------------------------------------------------------------------------
// The V part of split_qkv (decoder_compiler.cpp:116-148; V is not rotated)
// written transposed for the flash prefill: V^T [B][Hkv][128][ld_vt] bf16 with
// keys in [seq, ld_vt) zero.  One workgroup per (64-key block, kv_head, batch):
// the fp32 [64 keys][128 dims] block is staged in LDS, then written as 16-byte
// runs of 8 keys per dim row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void v_transpose_kernel(const float* __restrict__ qkv,
                                                         int64_t qkv_ld, int64_t v_col0, int seq,
                                                         int kv_heads, int ld_vt,
                                                         uint16_t* __restrict__ vt) {
    __shared__ float tile[64][129];
    const int s0 = blockIdx.x * 64;
    const int hkv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int idx = tid + 256 * it;
        const int key = idx >> 5, d4 = (idx & 31) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (s0 + key < seq)
            v = *reinterpret_cast<const float4*>(qkv + (static_cast<int64_t>(b) * seq + s0 + key) * qkv_ld +
                                                 v_col0 + hkv * 128 + d4);
        tile[key][d4] = v.x;
        tile[key][d4 + 1] = v.y;
        tile[key][d4 + 2] = v.z;
        tile[key][d4 + 3] = v.w;
    }
    __syncthreads();
    uint16_t* dst = vt + (static_cast<int64_t>(b) * kv_heads + hkv) * 128 * ld_vt + s0;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = tid + 256 * it;
        const int d = idx >> 3, k8 = (idx & 7) * 8;
        uint4 pk;
        pk.x = pack_bf16x2(tile[k8 + 0][d], tile[k8 + 1][d]);
        pk.y = pack_bf16x2(tile[k8 + 2][d], tile[k8 + 3][d]);
        pk.z = pack_bf16x2(tile[k8 + 4][d], tile[k8 + 5][d]);
        pk.w = pack_bf16x2(tile[k8 + 6][d], tile[k8 + 7][d]);
        *reinterpret_cast<uint4*>(dst + static_cast<int64_t>(d) * ld_vt + k8) = pk;
    }
}

void launch_v_transpose(const float* qkv, int64_t batch, int64_t seq, int64_t q_heads,
                        int64_t kv_heads, int64_t ld_vt, uint16_t* vt, hipStream_t stream) {
    const int64_t qkv_ld = (q_heads + 2 * kv_heads) * 128;
    const int64_t v_col0 = (q_heads + kv_heads) * 128;
    const dim3 grid(static_cast<unsigned>(ld_vt / 64), static_cast<unsigned>(kv_heads),
                    static_cast<unsigned>(batch));
    v_transpose_kernel<<<grid, 256, 0, stream>>>(qkv, qkv_ld, v_col0, static_cast<int>(seq),
                                                 static_cast<int>(kv_heads), static_cast<int>(ld_vt), vt);
}

// ---------------------------------------------------------------------------
// Weight packing: fp32 [K][N] -> [N][K] (fp32 or bf16) through a 64x64 LDS tile
// so both the read and the write are coalesced.
// ---------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(256) void transpose_pack_kernel(const float* __restrict__ src,
                                                             int64_t k, int64_t n, int64_t ld,
                                                             OutT* __restrict__ dst) {
    __shared__ float tile[64][65];
    const int64_t k0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int64_t kk = k0 + r, nn = n0 + tx;
        tile[r][tx] = (kk < k && nn < n) ? src[kk * ld + nn] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int64_t nn = n0 + r, kk = k0 + tx;
        if (nn < n && kk < k) {
            const float val = tile[tx][r];
            if constexpr (sizeof(OutT) == 4) dst[nn * k + kk] = val;
            else dst[nn * k + kk] = f32_to_bf16(val);
        }
    }
}

// Fragment-tiled packing (SFG_LAYOUT_TILED): one thread per 16-byte lane
// fragment.  bf16 tile = 16 rows x 128 k = 4 fragments x 64 lanes x 8 values;
// lane l = 16 g + r holds row r and k = 32 s + 8 g + [0, 8) of fragment s.
__global__ __launch_bounds__(256) void pack_tiled_bf16_kernel(const float* __restrict__ src,
                                                              int64_t k, int64_t n, int64_t ld,
                                                              uint16_t* __restrict__ dst) {
    const int64_t chunks = k / 128;
    const int64_t total = (n / 16) * chunks * 4 * 64;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int lane = static_cast<int>(idx & 63);
    const int s = static_cast<int>((idx >> 6) & 3);
    const int64_t tc = idx >> 8;
    const int64_t kc = tc % chunks, nt = tc / chunks;
    const int64_t col = nt * 16 + (lane & 15);
    const int64_t k0 = kc * 128 + 32 * s + 8 * (lane >> 4);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = src[(k0 + j) * ld + col];
    *reinterpret_cast<uint4*>(dst + idx * 8) = f32x8_to_bf16x8(v);
}

// int8 tile = 16 rows x 128 k = 2 fragments x 64 lanes x 16 values; lane
// l = 16 g + r holds row r and k = 32 g + 16 t + [0, 16) of fragment t.
__global__ __launch_bounds__(256) void quantize_tiled_kernel(const float* __restrict__ src,
                                                             int64_t k, int64_t n,
                                                             const float* __restrict__ scales,
                                                             int8_t* __restrict__ dst) {
    const int64_t chunks = k / 128;
    const int64_t total = (n / 16) * chunks * 2 * 64;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int lane = static_cast<int>(idx & 63);
    const int t = static_cast<int>((idx >> 6) & 1);
    const int64_t tc = idx >> 7;
    const int64_t kc = tc % chunks, nt = tc / chunks;
    const int64_t col = nt * 16 + (lane & 15);
    const int64_t k0 = kc * 128 + 32 * (lane >> 4) + 16 * t;
    const float sc = scales[col];
    int8_t q[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        float r = roundf(src[(k0 + j) * n + col] / sc);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        q[j] = static_cast<int8_t>(r);
    }
    *reinterpret_cast<uint4*>(dst + idx * 16) = *reinterpret_cast<const uint4*>(q);
}

void launch_pack_weight(const float* src, int64_t k, int64_t n, int64_t ld, void* dst,
                        int dtype, int layout, hipStream_t stream) {
    if (layout == SFG_LAYOUT_TILED) {
        const int64_t total = (n / 16) * (k / 128) * 256;
        pack_tiled_bf16_kernel<<<dim3(static_cast<unsigned>((total + 255) / 256)), 256, 0, stream>>>(
            src, k, n, ld, static_cast<uint16_t*>(dst));
        return;
    }
    const dim3 grid(static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>((k + 63) / 64));
    if (dtype == SFG_F32)
        transpose_pack_kernel<float><<<grid, 256, 0, stream>>>(src, k, n, ld,
                                                              static_cast<float*>(dst));
    else
        transpose_pack_kernel<uint16_t><<<grid, 256, 0, stream>>>(src, k, n, ld,
                                                                 static_cast<uint16_t*>(dst));
}

// quantize_matmul_weights (next_milestones.cpp:611-637) applied to the
// transposed weight (transpose_decoder_weight, 233-244).  Pass 1: one thread per
// output channel n walks its column of src [K][N] (coalesced across n) for the
// absmax.  Pass 2: the transposing tile kernel quantises.
__global__ __launch_bounds__(256) void column_absmax_kernel(const float* __restrict__ src,
                                                            int64_t k, int64_t n,
                                                            float* __restrict__ scales) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (col >= n) return;
    float maximum = 0.0f;
    for (int64_t r = 0; r < k; ++r) maximum = fmaxf(maximum, fabsf(src[r * n + col]));
    float scale = maximum > 0.0f ? maximum / 127.0f : 1.0f;
    if (scale == 0.0f) scale = 1.0f;
    scales[col] = scale;
}

__global__ __launch_bounds__(256) void quantize_pack_kernel(const float* __restrict__ src,
                                                            int64_t k, int64_t n,
                                                            const float* __restrict__ scales,
                                                            int8_t* __restrict__ dst) {
    __shared__ float tile[64][65];
    const int64_t k0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int64_t kk = k0 + r, nn = n0 + tx;
        tile[r][tx] = (kk < k && nn < n) ? src[kk * n + nn] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int64_t nn = n0 + r, kk = k0 + tx;
        if (nn < n && kk < k) {
            float q = roundf(tile[tx][r] / scales[nn]);
            q = fminf(fmaxf(q, -127.0f), 127.0f);
            dst[nn * k + kk] = static_cast<int8_t>(q);
        }
    }
}

void launch_quantize_weight(const float* src, int64_t k, int64_t n, int8_t* dst, float* scales,
                            int layout, hipStream_t stream) {
    column_absmax_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), 256, 0, stream>>>(
        src, k, n, scales);
    if (layout == SFG_LAYOUT_TILED) {
        const int64_t total = (n / 16) * (k / 128) * 128;
        quantize_tiled_kernel<<<dim3(static_cast<unsigned>((total + 255) / 256)), 256, 0, stream>>>(
            src, k, n, scales, dst);
        return;
    }
    const dim3 grid(static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>((k + 63) / 64));
    quantize_pack_kernel<<<grid, 256, 0, stream>>>(src, k, n, scales, dst);
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ src,
                                                      uint16_t* __restrict__ dst, int64_t count) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) dst[i] = f32_to_bf16(src[i]);
}

void launch_to_bf16(const float* src, uint16_t* dst, int64_t count, hipStream_t stream) {
    to_bf16_kernel<<<dim3(static_cast<unsigned>((count + 255) / 256)), 256, 0, stream>>>(
        src, dst, count);
}

// Zero-fill (used instead of hipMemsetAsync so the layer stays capturable).
__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t* __restrict__ dst, int64_t words) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < words) dst[i] = 0u;
}

void launch_fill_zero(void* dst, size_t bytes, hipStream_t stream) {
    const int64_t words = static_cast<int64_t>(bytes / 4);
    if (words == 0) return;
    fill_zero_kernel<<<dim3(static_cast<unsigned>((words + 255) / 256)), 256, 0, stream>>>(
        static_cast<uint32_t*>(dst), words);
}

}  // namespace sfg
