// sfg_api.hip -- the C ABI (include/sfg_hip.h) and the decoder-layer
// orchestration: the GPU counterpart of execute_once
// (decoder_compiler.cpp:218-304).
//
// Every entry point validates its arguments on the host before launching, so
// shape and guard violations come back as SFG_ERR_* codes (the reference's
// std::invalid_argument cases) instead of faults; HIP failures come back as
// SFG_ERR_DEVICE with the runtime's message.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "sfg_kernels.hpp"

// Library-held split partials of the paged decode, for callers that cannot
// allocate (sfg_hip_attn_decode_paged_noalloc_v1).  Each device holds its own
// copy from the library's load until the process ends.  Host code never uses
// this name as an address: the per-device address comes from
// hipGetSymbolAddress (scratch_on_current_device below).
static __device__ __align__(256) unsigned char scratch[SFG_DECODE_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(SFG_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
    return SFG_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

float default_scale(int64_t head_dim, float scale) {
    return scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
}

// Argument checks shared by the two paged-decode entry points.
int check_decode_args(const float* q, const void* k_pool, const void* v_pool,
                      const int32_t* page_table, const void* out, int64_t batch, int64_t q_heads,
                      int64_t kv_heads, int64_t head_dim, int64_t page_tokens, int64_t pages_per_seq,
                      int64_t num_pages, int64_t max_context) {
    if (!q || !k_pool || !v_pool || !page_table || !out || batch <= 0 || q_heads <= 0 ||
        kv_heads <= 0 || q_heads % kv_heads || head_dim <= 0 || page_tokens <= 0 ||
        pages_per_seq <= 0 || num_pages <= 0 || max_context <= 0)
        return fail(SFG_ERR_INVALID_CONFIG, "attn_decode_paged: invalid configuration");
    if (max_context > pages_per_seq * page_tokens)
        return fail(SFG_ERR_GUARD, "paged KV length violates compiled guard (%lld > %lld)",
                    (long long)max_context, (long long)(pages_per_seq * page_tokens));
    if (head_dim > 256) return fail(SFG_ERR_UNSUPPORTED, "paged attention: head_dim %lld > 256", (long long)head_dim);
    return SFG_OK;
}

// Which decode kernel a paged-attention call runs and its split count: the
// MFMA split-KV kernel where it lowers the shape, else the row kernel (any
// head_dim <= 256, page size, new-token count and pool dtype).  `bytes` is
// the partials' workspace.
struct DecodePlan {
    bool mfma;
    int splits;
    size_t bytes;
};

DecodePlan plan_decode(int kv_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                       int64_t head_dim, int64_t page_tokens, int64_t max_context, int32_t kv_splits) {
    if (sfg::decode_mfma_supported(kv_dtype, head_dim, page_tokens, q_heads / kv_heads, seq_q)) {
        const int s = sfg::decode_split_count(batch, kv_heads, max_context, page_tokens, kv_splits);
        return {true, s, sfg::decode_workspace_bytes(batch, q_heads, head_dim, s)};
    }
    const int64_t rows = batch * seq_q * q_heads;
    const int s = sfg::paged_rows_split_count(rows, max_context, kv_splits);
    return {false, s, sfg::paged_rows_workspace_bytes(rows, head_dim, s)};
}

// The paged attention of the standalone entry points: Q and the output
// head-major [B][Hq][Sq][D] (one row per (b, h) when Sq = 1, which is also the
// MFMA kernel's [B][Hq * D]), partials in ws.
int launch_paged(const DecodePlan& plan, const float* q, const void* k_pool, const void* v_pool,
                 int kv_dtype, const int32_t* page_table, const int32_t* seq_lens, void* out,
                 int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                 int64_t head_dim, int64_t page_tokens, int64_t pages_per_seq, int64_t num_pages,
                 int64_t max_context, int causal, float scale, void* ws, void* stream) {
    const float sc = default_scale(head_dim, scale);
    int rc;
    if (plan.mfma) {
        rc = sfg::launch_attn_decode_paged(
            q, q_heads * head_dim, nullptr, 0, static_cast<const uint16_t*>(k_pool),
            static_cast<const uint16_t*>(v_pool), page_table, seq_lens, max_context, 0, out, out_dtype,
            batch, q_heads, kv_heads, head_dim, page_tokens, pages_per_seq, num_pages, plan.splits, sc,
            ws, as_stream(stream), nullptr);
    } else {
        sfg::PagedRowsLaunch a{};
        a.q = q;
        a.q_stride_b = q_heads * seq_q * head_dim; a.q_stride_i = head_dim; a.q_stride_h = seq_q * head_dim;
        a.k_pool = k_pool; a.v_pool = v_pool; a.kv_dtype = kv_dtype;
        a.page_table = page_table; a.seq_lens = seq_lens; a.max_context = max_context;
        a.out = out; a.out_dtype = out_dtype;
        a.out_stride_b = a.q_stride_b; a.out_stride_i = a.q_stride_i; a.out_stride_h = a.q_stride_h;
        a.batch = batch; a.q_heads = q_heads; a.kv_heads = kv_heads; a.seq_q = seq_q;
        a.head_dim = head_dim; a.page_tokens = page_tokens; a.pages_per_seq = pages_per_seq;
        a.num_pages = num_pages; a.splits = plan.splits; a.causal = causal; a.scale = sc;
        rc = sfg::launch_attn_paged_rows(a, ws, as_stream(stream));
    }
    if (rc != SFG_OK)
        return fail(rc, "paged attention: head_dim %lld / page_tokens %lld / group %lld not lowered",
                    (long long)head_dim, (long long)page_tokens, (long long)(q_heads / kv_heads));
    return check_launch("paged attention");
}

// Host-side page-id validation (validate_pages): the table read back and every
// used entry checked against the pool.
int validate_page_ids(const int32_t* page_table, int64_t batch, int64_t pages_per_seq, int64_t num_pages,
                      int64_t max_context, int64_t page_tokens, void* stream) {
    std::vector<int32_t> table(static_cast<size_t>(batch * pages_per_seq));
    hipError_t e = hipMemcpyAsync(table.data(), page_table, table.size() * sizeof(int32_t),
                                  hipMemcpyDeviceToHost, as_stream(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
    if (e != hipSuccess) return fail(SFG_ERR_DEVICE, "page table readback: %s", hipGetErrorString(e));
    const int64_t used = (max_context + page_tokens - 1) / page_tokens;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t p = 0; p < used; ++p) {
            const int32_t id = table[static_cast<size_t>(b * pages_per_seq + p)];
            if (id < 0 || id >= num_pages)
                return fail(SFG_ERR_GUARD, "invalid physical KV page %d (sequence %lld, page %lld)",
                            id, (long long)b, (long long)p);
        }
    return SFG_OK;
}

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(SFG_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(SFG_ERR_UNSUPPORTED, "device %d beyond the %d the library tracks", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(SFG_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return SFG_OK;
}

}  // namespace

namespace sfg {

int device_xcds(hipStream_t stream) {
    // One query per device, kept in a lock-free table: concurrent first calls
    // store the same value.  The device is the stream's (the null stream's is
    // the current device), so a call with another device's stream gets that
    // device's count.
    static std::atomic<int> cache[kMaxDevices];
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 1;
    int x = cache[dev].load(std::memory_order_relaxed);
    if (x == 0) {
        if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x <= 0) x = 1;
        cache[dev].store(x, std::memory_order_relaxed);
    }
    return x;
}

int device_cus(hipStream_t stream) {
    // Compute units of the stream's device, cached like device_xcds.
    static std::atomic<int> cache[kMaxDevices];
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 1;
    int x = cache[dev].load(std::memory_order_relaxed);
    if (x == 0) {
        if (hipDeviceGetAttribute(&x, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || x <= 0) x = 1;
        cache[dev].store(x, std::memory_order_relaxed);
    }
    return x;
}

}  // namespace sfg

namespace {

// Bump allocator over the caller's workspace.
struct Carve {
    char* base;
    size_t used = 0;
    explicit Carve(void* b) : base(static_cast<char*>(b)) {}
    void* take(size_t bytes) {
        void* p = base ? base + used : nullptr;
        used += align256(bytes);
        return p;
    }
};

}  // namespace

extern "C" {

int sfg_hip_abi_version(void) { return SFG_HIP_ABI_VERSION; }

// The lowering envelope, key=value pairs separated by ';' (after the
// reference's schedforge_aot_metadata_v1 invariants, llvm_backend.cpp:622-643):
//   act / weights          activation dtypes and the weight dtypes each takes
//   kv                     paged pools hold the activation dtype
//   head_dim, page_tokens, decode_tokens   the widest shapes any path lowers
//   mfma_*                 the shapes the MFMA kernels take (everything else
//                          runs the row-per-wave attention / VALU GEMM paths)
const char* sfg_hip_metadata_v1(void) {
    return "abi=1;arch=gfx950;wavefront=64;dtypes=f32,bf16,i8;act=f32,bf16;"
           "weights=f32:f32,bf16:bf16|i8;weight_layout=NK,TILED;"
           "kv_layout=page,kv_head,page_token,head_dim;kv=act_dtype;"
           "head_dim=1..256;page_tokens=any;decode_tokens=any;ffn=dense,moe;"
           "mfma_decode=bf16,head_dim=64|128,page_tokens=16,decode_tokens=1,gqa_group=1|2|4|8|16;"
           "mfma_prefill=bf16,head_dim=64|128;mfma_gemm=bf16|i8,k%32==0;"
           "accumulate=f32;bf16_rounding=rne";
}

const char* sfg_hip_last_error(void) { return g_last_error.c_str(); }

int sfg_hip_device_info_v1(int device, int* cu_count, int* xcd_count, int64_t* hbm_bytes) {
    sfg_target_info t;
    const int rc = sfg_hip_target_info_v1(device, &t);
    if (rc != SFG_OK) return rc;
    if (cu_count) *cu_count = t.compute_units;
    if (xcd_count) *xcd_count = t.xcds;
    if (hbm_bytes) *hbm_bytes = t.hbm_bytes;
    return SFG_OK;
}

int sfg_hip_target_info_v1(int device, sfg_target_info* info) {
    if (!info) return fail(SFG_ERR_SHAPE, "target_info: null output");
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(SFG_ERR_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    // A runtime that cannot report XCDs gets one, as the kernel launches
    // assume (device_xcds): the query still describes the device.
    int xcds = 0;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, device) != hipSuccess) xcds = 1;
    sfg_target_info t{};
    snprintf(t.architecture, sizeof t.architecture, "%s", prop.gcnArchName);
    t.wavefront = prop.warpSize;
    t.compute_units = prop.multiProcessorCount;
    t.xcds = xcds > 0 ? xcds : 1;
    t.simds_per_cu = 4;
    t.lds_bytes_per_cu = static_cast<int64_t>(prop.maxSharedMemoryPerMultiProcessor);
    // HIP reports no L2 size for this architecture (prop.l2CacheSize is 0 or
    // the whole device's); gfx950 has 4 MiB per XCD.
    t.l2_bytes_per_xcd = prop.l2CacheSize > 0 && prop.l2CacheSize / t.xcds >= (1 << 20)
                             ? prop.l2CacheSize / t.xcds : (int64_t(4) << 20);
    t.hbm_bytes = static_cast<int64_t>(prop.totalGlobalMem);
    t.engine_clock_ghz = prop.clockRate / 1.0e6;
    // HIP's memory clock times two transfers per clock over the bus width
    // understates HBM3E (on MI355X it reads 4.1 TB/s, half the 8 GT/s pin
    // rate), so gfx950 takes its published 8 TB/s; other parts the estimate.
    t.hbm_gbps = strncmp(prop.gcnArchName, "gfx950", 6) == 0
                     ? 8000.0
                     : 2.0 * prop.memoryClockRate * 1.0e3 * (prop.memoryBusWidth / 8.0) / 1.0e9;
    t.mfma_bf16_tflops = t.compute_units * 4096.0 * t.engine_clock_ghz / 1.0e3;
    t.valu_fp32_tflops = t.compute_units * 256.0 * t.engine_clock_ghz / 1.0e3;
    *info = t;
    return SFG_OK;
}

static int check_layout(int layout, int64_t k, int64_t n, const char* what) {
    if (layout != SFG_LAYOUT_NK && layout != SFG_LAYOUT_TILED)
        return fail(SFG_ERR_SHAPE, "%s: unknown layout %d", what, layout);
    if (layout == SFG_LAYOUT_TILED && (n % 16 != 0 || k % 128 != 0))
        return fail(SFG_ERR_SHAPE, "%s: tiled layout needs N %% 16 == 0 and K %% 128 == 0 (N=%lld K=%lld)",
                    what, (long long)n, (long long)k);
    return SFG_OK;
}

int sfg_hip_pack_weight_v1(const float* src, int64_t k, int64_t n, int64_t ld_src, void* dst,
                           int dst_dtype, int layout, void* stream) {
    if (!src || !dst || k <= 0 || n <= 0 || ld_src < n)
        return fail(SFG_ERR_SHAPE, "pack_weight: invalid arguments k=%lld n=%lld ld=%lld",
                    (long long)k, (long long)n, (long long)ld_src);
    if (dst_dtype != SFG_F32 && dst_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "pack_weight: dtype %d", dst_dtype);
    int rc = check_layout(layout, k, n, "pack_weight");
    if (rc) return rc;
    if (layout == SFG_LAYOUT_TILED && dst_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "pack_weight: tiled layout is bf16 / int8 only");
    sfg::launch_pack_weight(src, k, n, ld_src, dst, dst_dtype, layout, as_stream(stream));
    return check_launch("pack_weight");
}

int sfg_hip_quantize_weight_v1(const float* src, int64_t k, int64_t n, int8_t* dst,
                               float* scales, int layout, void* stream) {
    if (!src || !dst || !scales || k <= 0 || n <= 0)
        return fail(SFG_ERR_SHAPE, "quantize_weight: invalid arguments");
    int rc = check_layout(layout, k, n, "quantize_weight");
    if (rc) return rc;
    sfg::launch_quantize_weight(src, k, n, dst, scales, layout, as_stream(stream));
    return check_launch("quantize_weight");
}

int sfg_hip_preferred_weight_layout_v1(int64_t rows, int64_t k, int grouped) {
    return sfg::gemm_preferred_layout(rows, k, grouped != 0);
}

int sfg_hip_to_bf16_v1(const float* src, uint16_t* dst, int64_t count, void* stream) {
    if (count < 0 || (count > 0 && (!src || !dst))) return fail(SFG_ERR_SHAPE, "to_bf16: invalid");
    if (count == 0) return SFG_OK;
    sfg::launch_to_bf16(src, dst, count, as_stream(stream));
    return check_launch("to_bf16");
}

int sfg_hip_rope_table_host_v1(float* table, int64_t seq, int64_t head_dim, float theta) {
    // [seq][head_dim / 2][cos, sin]: an odd head_dim's last dimension is not
    // rotated (apply_rope's loop stops at dimension + 1 < head_dim)
    if (seq <= 0 || head_dim <= 0 || (!table && head_dim >= 2))
        return fail(SFG_ERR_SHAPE, "rope_table: invalid arguments");
    // The reference's expressions (decoder_compiler.cpp:101-106), evaluated
    // with the host libm: f = powf(theta, -float(2i)/float(D)); a = float(pos) * f.
    for (int64_t s = 0; s < seq; ++s)
        for (int64_t i = 0; i < head_dim / 2; ++i) {
            const float freq = powf(theta, -static_cast<float>(2 * i) / static_cast<float>(head_dim));
            const float angle = static_cast<float>(s) * freq;
            table[(s * (head_dim / 2) + i) * 2] = cosf(angle);
            table[(s * (head_dim / 2) + i) * 2 + 1] = sinf(angle);
        }
    return SFG_OK;
}

int sfg_hip_rmsnorm_v1(const float* x, const float* w, void* y, int y_dtype, int64_t rows,
                       int64_t width, float eps, void* stream) {
    if (!x || !w || !y || rows <= 0 || width <= 0 || !(eps > 0.0f))
        return fail(SFG_ERR_SHAPE, "rmsnorm: invalid arguments");
    if (y_dtype != SFG_F32 && y_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "rmsnorm: dtype %d", y_dtype);
    sfg::launch_rmsnorm(x, w, y, y_dtype, rows, width, eps, as_stream(stream));
    return check_launch("rmsnorm");
}

size_t sfg_hip_gemm_workspace_v1(int64_t m, int64_t n, int64_t k) {
    return sfg::gemm_workspace_bytes(m, 2 * n, k);
}

int sfg_hip_gemm_v1(const sfg_gemm_args* a, void* workspace, size_t workspace_bytes, void* stream) {
    if (!a || !a->a || !a->b || !a->c || a->m <= 0 || a->n <= 0 || a->k <= 0)
        return fail(SFG_ERR_SHAPE, "gemm: invalid arguments");
    if (a->lda < a->k || a->ldb < a->k)
        return fail(SFG_ERR_SHAPE, "gemm: leading dimension smaller than k");
    const bool glu = a->epilogue == SFG_EPI_SWIGLU || a->epilogue == SFG_EPI_GLU_SILU_UP;
    if (a->ldc < a->n) return fail(SFG_ERR_SHAPE, "gemm: ldc < n");
    if (a->epilogue == SFG_EPI_RESIDUAL && (!a->residual || a->ldr < a->n))
        return fail(SFG_ERR_SHAPE, "gemm: residual epilogue needs residual [m][n]");
    if (a->epilogue < SFG_EPI_NONE || a->epilogue > SFG_EPI_GLU_SILU_UP)
        return fail(SFG_ERR_SHAPE, "gemm: unknown epilogue %d", a->epilogue);
    (void)glu;
    sfg::GemmProblem p{};
    p.a = a->a; p.a_dtype = a->a_dtype; p.lda = a->lda; p.a_rows = nullptr;
    p.b = a->b; p.b_dtype = a->b_dtype; p.ldb = a->ldb; p.b_scales = a->b_scales;
    p.c = a->c; p.c_dtype = a->c_dtype; p.ldc = a->ldc;
    p.residual = a->residual; p.ldr = a->ldr;
    p.m = a->m; p.n = a->n; p.k = a->k; p.epilogue = a->epilogue;
    p.b_layout = a->b_layout;
    p.offsets = nullptr; p.groups = 1;
    p.tile = a->tile;
    if (a->b_layout != SFG_LAYOUT_NK && a->b_layout != SFG_LAYOUT_TILED)
        return fail(SFG_ERR_SHAPE, "gemm: unknown weight layout %d", a->b_layout);
    if (a->tile < SFG_TILE_AUTO || a->tile >= SFG_TILE_COUNT)
        return fail(SFG_ERR_SHAPE, "gemm: unknown tile policy %d", a->tile);
    const int rc = sfg::launch_gemm(p, workspace, workspace_bytes, as_stream(stream));
    if (rc != SFG_OK)
        return fail(rc, "gemm: unsupported or invalid combination (a=%d b=%d m=%lld n=%lld k=%lld epi=%d)",
                    a->a_dtype, a->b_dtype, (long long)a->m, (long long)a->n, (long long)a->k,
                    a->epilogue);
    return check_launch("gemm");
}

int sfg_hip_gemm_grouped_v1(const sfg_gemm_args* a, const int32_t* a_rows, int64_t a_rows_limit,
                            const int32_t* offsets, int groups, int64_t b_group_stride,
                            int64_t s_group_stride, void* workspace, size_t workspace_bytes,
                            void* stream) {
    (void)workspace; (void)workspace_bytes;  // grouped products reduce inside their workgroups
    if (!a || !a->a || !a->b || !a->c || !offsets || a->m <= 0 || a->n <= 0 || a->k <= 0 || groups <= 0)
        return fail(SFG_ERR_SHAPE, "gemm_grouped: invalid arguments");
    if (a->lda < a->k || a->ldb < a->k || a->ldc < a->n)
        return fail(SFG_ERR_SHAPE, "gemm_grouped: leading dimension too small");
    if (a_rows && a_rows_limit <= 0) return fail(SFG_ERR_SHAPE, "gemm_grouped: a_rows_limit must be > 0");
    if (a->epilogue == SFG_EPI_RESIDUAL || a->epilogue < SFG_EPI_NONE || a->epilogue > SFG_EPI_GLU_SILU_UP)
        return fail(SFG_ERR_SHAPE, "gemm_grouped: epilogue %d (none, SwiGLU or GLU)", a->epilogue);
    if (a->b_layout != SFG_LAYOUT_NK && a->b_layout != SFG_LAYOUT_TILED)
        return fail(SFG_ERR_SHAPE, "gemm_grouped: unknown weight layout %d", a->b_layout);
    if (a->tile < SFG_TILE_AUTO || a->tile >= SFG_TILE_COUNT)
        return fail(SFG_ERR_SHAPE, "gemm_grouped: unknown tile policy %d", a->tile);
    sfg::GemmProblem p{};
    p.a = a->a; p.a_dtype = a->a_dtype; p.lda = a->lda; p.a_rows = a_rows;
    p.a_rows_limit = a_rows ? a_rows_limit : a->m;
    p.b = a->b; p.b_dtype = a->b_dtype; p.ldb = a->ldb; p.b_scales = a->b_scales;
    p.b_group_stride = b_group_stride; p.s_group_stride = s_group_stride;
    p.c = a->c; p.c_dtype = a->c_dtype; p.ldc = a->ldc;
    p.m = a->m; p.n = a->n; p.k = a->k; p.epilogue = a->epilogue;
    p.b_layout = a->b_layout; p.offsets = offsets; p.groups = groups; p.tile = a->tile;
    const int rc = sfg::launch_gemm(p, nullptr, 0, as_stream(stream));
    if (rc != SFG_OK)
        return fail(rc, "gemm_grouped: unsupported combination (a=%d b=%d m=%lld n=%lld k=%lld epi=%d)",
                    a->a_dtype, a->b_dtype, (long long)a->m, (long long)a->n, (long long)a->k, a->epilogue);
    return check_launch("gemm_grouped");
}

int sfg_hip_qkv_split_rope_v1(const float* qkv, const float* rope_table, int64_t batch,
                              int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                              void* q, void* k, void* v, int out_dtype, void* stream) {
    // any head_dim: an odd one's last dimension is copied unrotated, as
    // apply_rope's pair loop (d + 1 < head_dim) leaves it; head_dim 1 has no
    // pair and reads no table
    if (!qkv || (!rope_table && head_dim >= 2) || !q || batch <= 0 || seq <= 0 || q_heads <= 0 ||
        kv_heads <= 0 || head_dim <= 0 || q_heads % kv_heads)
        return fail(SFG_ERR_SHAPE, "qkv_split_rope: invalid arguments");
    if (out_dtype != SFG_F32 && out_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "qkv_split_rope: dtype %d", out_dtype);
    sfg::launch_split_rope(qkv, rope_table, batch, seq, q_heads, kv_heads, head_dim, q, k, v,
                           out_dtype, as_stream(stream));
    return check_launch("qkv_split_rope");
}

int sfg_hip_attn_prefill_v1(const void* q, const void* k, const void* v, void* out, int dtype,
                            int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                            int64_t seq_q, int64_t seq_kv, int64_t head_dim, int causal,
                            float scale, void* stream) {
    // validate_config (attention_compiler.cpp:23-29)
    if (!q || !k || !v || !out || batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq_q <= 0 ||
        seq_kv <= 0 || head_dim <= 0 || q_heads % kv_heads || (causal && seq_q > seq_kv))
        return fail(SFG_ERR_INVALID_CONFIG, "invalid attention configuration");
    const float s = default_scale(head_dim, scale);
    if (dtype == SFG_F32) {
        const int rc = sfg::launch_attn_prefill_f32(
            static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
            out, out_dtype, batch, q_heads, kv_heads, seq_q, seq_kv, head_dim, causal, s,
            as_stream(stream));
        if (rc != SFG_OK) return fail(rc, "attn_prefill f32: head_dim %lld > 256", (long long)head_dim);
    } else if (dtype == SFG_BF16) {
        const int rc = sfg::launch_attn_prefill_bf16(
            static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
            static_cast<const uint16_t*>(v), out, out_dtype, batch, q_heads, kv_heads, seq_q,
            seq_kv, head_dim, causal, s, as_stream(stream));
        if (rc != SFG_OK) return fail(rc, "attn_prefill bf16: head_dim %lld not lowered", (long long)head_dim);
    } else {
        return fail(SFG_ERR_UNSUPPORTED, "attn_prefill: dtype %d", dtype);
    }
    return check_launch("attn_prefill");
}

int64_t sfg_hip_attn_vt_ld_v1(int64_t seq_kv) { return seq_kv > 0 ? sfg::attn_vt_ld(seq_kv) : 0; }

int sfg_hip_qkv_split_rope_vt_v1(const float* qkv, const float* rope_table, int64_t batch,
                                 int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                 uint16_t* q, uint16_t* k, uint16_t* vt, int64_t ld_vt,
                                 void* stream) {
    if (!qkv || !rope_table || !q || !k || !vt || batch <= 0 || seq <= 0 || q_heads <= 0 ||
        kv_heads <= 0 || q_heads % kv_heads)
        return fail(SFG_ERR_SHAPE, "qkv_split_rope_vt: invalid arguments");
    if (head_dim != 128) return fail(SFG_ERR_UNSUPPORTED, "qkv_split_rope_vt: head_dim %lld", (long long)head_dim);
    if (ld_vt != sfg::attn_vt_ld(seq))
        return fail(SFG_ERR_SHAPE, "qkv_split_rope_vt: ld_vt %lld != %lld", (long long)ld_vt,
                    (long long)sfg::attn_vt_ld(seq));
    const hipStream_t s = as_stream(stream);
    sfg::launch_split_rope(qkv, rope_table, batch, seq, q_heads, kv_heads, head_dim, q, k, nullptr,
                           SFG_BF16, s);
    sfg::launch_v_transpose(qkv, batch, seq, q_heads, kv_heads, ld_vt, vt, s);
    return check_launch("qkv_split_rope_vt");
}

int sfg_hip_attn_prefill_vt_v1(const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                               int64_t ld_vt, void* out, int out_dtype, int64_t batch,
                               int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_kv,
                               int64_t head_dim, int causal, float scale, void* stream) {
    if (!q || !k || !vt || !out || batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq_q <= 0 ||
        seq_kv <= 0 || head_dim <= 0 || q_heads % kv_heads || (causal && seq_q > seq_kv))
        return fail(SFG_ERR_INVALID_CONFIG, "invalid attention configuration");
    if (out_dtype != SFG_F32 && out_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "attn_prefill_vt: out dtype %d", out_dtype);
    if (ld_vt != sfg::attn_vt_ld(seq_kv))
        return fail(SFG_ERR_SHAPE, "attn_prefill_vt: ld_vt %lld != %lld", (long long)ld_vt,
                    (long long)sfg::attn_vt_ld(seq_kv));
    const int rc = sfg::launch_attn_prefill_vt(q, k, vt, ld_vt, out, out_dtype, batch, q_heads,
                                               kv_heads, seq_q, seq_kv, head_dim, causal,
                                               default_scale(head_dim, scale), 0, as_stream(stream));
    if (rc != SFG_OK) return fail(rc, "attn_prefill_vt: head_dim %lld not lowered", (long long)head_dim);
    return check_launch("attn_prefill_vt");
}

size_t sfg_hip_attn_decode_workspace_v1(int64_t batch, int64_t q_heads, int64_t head_dim,
                                        int64_t max_context, int64_t page_tokens,
                                        int32_t kv_splits) {
    // kv_heads only bounds the MFMA kernel's automatic split choice from
    // below; kv_heads = q_heads gives an upper bound on the split count chosen
    // for any kv_heads.  The row kernel's partials (shapes the MFMA kernel does
    // not lower) are covered too.
    if (batch <= 0 || q_heads <= 0 || head_dim <= 0 || max_context <= 0 || page_tokens <= 0) return 0;
    const int s = sfg::decode_split_count(batch, 1, max_context, page_tokens, kv_splits);
    const size_t mfma = sfg::decode_workspace_bytes(batch, q_heads, head_dim, s);
    const int rs = sfg::paged_rows_split_count(batch * q_heads, max_context, kv_splits);
    const size_t rows = sfg::paged_rows_workspace_bytes(batch * q_heads, head_dim, rs);
    return mfma > rows ? mfma : rows;
}

int sfg_hip_attn_decode_paged_v1(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                                 const int32_t* page_table, const int32_t* seq_lens, void* out,
                                 int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                 int64_t head_dim, int64_t page_tokens, int64_t pages_per_seq,
                                 int64_t num_pages, int64_t max_context, int32_t kv_splits,
                                 float scale, int validate_pages, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    int rc = check_decode_args(q, k_pool, v_pool, page_table, out, batch, q_heads, kv_heads, head_dim,
                               page_tokens, pages_per_seq, num_pages, max_context);
    if (rc != SFG_OK) return rc;
    if (validate_pages &&
        (rc = validate_page_ids(page_table, batch, pages_per_seq, num_pages, max_context, page_tokens,
                                stream)) != SFG_OK)
        return rc;
    const DecodePlan plan = plan_decode(SFG_BF16, batch, q_heads, kv_heads, 1, head_dim, page_tokens,
                                        max_context, kv_splits);
    if (plan.bytes > 0 && (!workspace || workspace_bytes < plan.bytes))
        return fail(SFG_ERR_WORKSPACE, "attn_decode_paged: workspace %zu < %zu", workspace_bytes, plan.bytes);
    return launch_paged(plan, q, k_pool, v_pool, SFG_BF16, page_table, seq_lens, out, out_dtype, batch,
                        q_heads, kv_heads, 1, head_dim, page_tokens, pages_per_seq, num_pages, max_context,
                        1, scale, workspace, stream);
}

int sfg_hip_attn_decode_paged_noalloc_v1(const float* q, const uint16_t* k_pool,
                                         const uint16_t* v_pool, const int32_t* page_table,
                                         const int32_t* seq_lens, void* out, int out_dtype,
                                         int64_t batch, int64_t q_heads, int64_t kv_heads,
                                         int64_t head_dim, int64_t page_tokens,
                                         int64_t pages_per_seq, int64_t num_pages,
                                         int64_t max_context, int32_t kv_splits, float scale,
                                         void* stream) {
    int rc = check_decode_args(q, k_pool, v_pool, page_table, out, batch, q_heads, kv_heads, head_dim,
                               page_tokens, pages_per_seq, num_pages, max_context);
    if (rc != SFG_OK) return rc;
    const DecodePlan plan = plan_decode(SFG_BF16, batch, q_heads, kv_heads, 1, head_dim, page_tokens,
                                        max_context, kv_splits);
    if (plan.bytes > SFG_DECODE_SCRATCH_BYTES)
        return fail(SFG_ERR_WORKSPACE,
                    "attn_decode_paged_noalloc: %zu bytes of split partials (batch %lld x %lld heads x "
                    "%d splits) exceed the library's %zu-byte scratch; use sfg_hip_attn_decode_paged_v1 "
                    "with a workspace",
                    plan.bytes, (long long)batch, (long long)q_heads, plan.splits,
                    (size_t)SFG_DECODE_SCRATCH_BYTES);
    void* ws = nullptr;
    if ((rc = scratch_on_current_device(&ws)) != SFG_OK) return rc;
    return launch_paged(plan, q, k_pool, v_pool, SFG_BF16, page_table, seq_lens, out, out_dtype, batch,
                        q_heads, kv_heads, 1, head_dim, page_tokens, pages_per_seq, num_pages, max_context,
                        1, scale, ws, stream);
}

size_t sfg_hip_attn_paged_workspace_v1(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                       int64_t seq_q, int64_t head_dim, int kv_dtype,
                                       int64_t max_context, int64_t page_tokens, int32_t kv_splits) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || seq_q <= 0 ||
        head_dim <= 0 || max_context <= 0 || page_tokens <= 0)
        return 0;
    return plan_decode(kv_dtype, batch, q_heads, kv_heads, seq_q, head_dim, page_tokens, max_context,
                       kv_splits).bytes;
}

int sfg_hip_attn_paged_v1(const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                          const int32_t* page_table, const int32_t* seq_lens, void* out, int out_dtype,
                          int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                          int64_t head_dim, int64_t page_tokens, int64_t pages_per_seq,
                          int64_t num_pages, int64_t max_context, int causal, int32_t kv_splits,
                          float scale, int validate_pages, void* workspace, size_t workspace_bytes,
                          void* stream) {
    int rc = check_decode_args(q, k_pool, v_pool, page_table, out, batch, q_heads, kv_heads, head_dim,
                               page_tokens, pages_per_seq, num_pages, max_context);
    if (rc != SFG_OK) return rc;
    // validate_config (attention_compiler.cpp:23-29): a causal query block no
    // longer than the keys it attends over
    if (seq_q <= 0 || (causal && seq_q > max_context))
        return fail(SFG_ERR_INVALID_CONFIG, "invalid attention configuration");
    if (kv_dtype != SFG_F32 && kv_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "paged attention: pool dtype %d", kv_dtype);
    if (out_dtype != SFG_F32 && out_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "paged attention: output dtype %d", out_dtype);
    if (validate_pages &&
        (rc = validate_page_ids(page_table, batch, pages_per_seq, num_pages, max_context, page_tokens,
                                stream)) != SFG_OK)
        return rc;
    const DecodePlan plan = plan_decode(kv_dtype, batch, q_heads, kv_heads, seq_q, head_dim, page_tokens,
                                        max_context, kv_splits);
    if (plan.bytes > 0 && (!workspace || workspace_bytes < plan.bytes))
        return fail(SFG_ERR_WORKSPACE, "attn_paged: workspace %zu < %zu", workspace_bytes, plan.bytes);
    return launch_paged(plan, q, k_pool, v_pool, kv_dtype, page_table, seq_lens, out, out_dtype, batch,
                        q_heads, kv_heads, seq_q, head_dim, page_tokens, pages_per_seq, num_pages,
                        max_context, causal, scale, workspace, stream);
}

int sfg_hip_kv_append_pool_v1(const void* keys, const void* values, int dtype, void* k_pool,
                              void* v_pool, int pool_dtype, const int32_t* page_table,
                              int32_t* seq_lens, int64_t start, int advance, int64_t batch,
                              int64_t kv_heads, int64_t tokens, int64_t head_dim, int64_t page_tokens,
                              int64_t pages_per_seq, int64_t num_pages, void* stream) {
    if (!keys || !values || !k_pool || !v_pool || !page_table || batch <= 0 || kv_heads <= 0 ||
        tokens <= 0 || head_dim <= 0 || page_tokens <= 0 || pages_per_seq <= 0 || num_pages <= 0)
        return fail(SFG_ERR_SHAPE, "kv_append: invalid arguments");
    if (dtype != SFG_F32 && dtype != SFG_BF16) return fail(SFG_ERR_UNSUPPORTED, "kv_append: dtype %d", dtype);
    if (pool_dtype != SFG_F32 && pool_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "kv_append: pool dtype %d", pool_dtype);
    if (!seq_lens && (start < 0 || start + tokens > pages_per_seq * page_tokens))
        return fail(SFG_ERR_GUARD, "paged KV capacity exceeded (%lld + %lld > %lld)", (long long)start,
                    (long long)tokens, (long long)(pages_per_seq * page_tokens));
    const int rc = sfg::launch_kv_append(keys, values, dtype, kv_heads * tokens * head_dim,
                                         tokens * head_dim, head_dim, nullptr, k_pool, v_pool, pool_dtype,
                                         page_table, seq_lens, start, advance, batch, kv_heads, tokens,
                                         head_dim, page_tokens, pages_per_seq, num_pages, as_stream(stream));
    if (rc != SFG_OK) return fail(rc, "kv_append: head_dim %lld / page_tokens %lld not lowered",
                                  (long long)head_dim, (long long)page_tokens);
    return check_launch("kv_append");
}

int sfg_hip_kv_append_paged_v1(const void* keys, const void* values, int dtype, uint16_t* k_pool,
                               uint16_t* v_pool, const int32_t* page_table, int32_t* seq_lens,
                               int64_t start, int advance, int64_t batch, int64_t kv_heads,
                               int64_t tokens, int64_t head_dim, int64_t page_tokens,
                               int64_t pages_per_seq, int64_t num_pages, void* stream) {
    return sfg_hip_kv_append_pool_v1(keys, values, dtype, k_pool, v_pool, SFG_BF16, page_table, seq_lens,
                                     start, advance, batch, kv_heads, tokens, head_dim, page_tokens,
                                     pages_per_seq, num_pages, stream);
}

int sfg_hip_kv_gather_pool_v1(const void* k_pool, const void* v_pool, int pool_dtype,
                              const int32_t* page_table, int64_t batch, int64_t kv_heads,
                              int64_t length, int64_t head_dim, int64_t page_tokens,
                              int64_t pages_per_seq, int64_t num_pages, float* keys, float* values,
                              void* stream) {
    if (!k_pool || !v_pool || !page_table || !keys || !values || batch <= 0 || kv_heads <= 0 ||
        head_dim <= 0 || page_tokens <= 0 || pages_per_seq <= 0 || num_pages <= 0)
        return fail(SFG_ERR_SHAPE, "kv_gather: invalid arguments");
    if (length <= 0) return fail(SFG_ERR_INVALID_CONFIG, "cannot gather empty paged KV cache");
    if (length > pages_per_seq * page_tokens)
        return fail(SFG_ERR_GUARD, "kv_gather: length %lld beyond the page table", (long long)length);
    if (pool_dtype != SFG_F32 && pool_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "kv_gather: pool dtype %d", pool_dtype);
    const int rc = sfg::launch_kv_gather(k_pool, v_pool, pool_dtype, page_table, batch, kv_heads, length,
                                         head_dim, page_tokens, pages_per_seq, num_pages, keys, values,
                                         as_stream(stream));
    if (rc != SFG_OK) return fail(rc, "kv_gather: head_dim %lld not lowered", (long long)head_dim);
    return check_launch("kv_gather");
}

int sfg_hip_kv_gather_paged_v1(const uint16_t* k_pool, const uint16_t* v_pool,
                               const int32_t* page_table, int64_t batch, int64_t kv_heads,
                               int64_t length, int64_t head_dim, int64_t page_tokens,
                               int64_t pages_per_seq, int64_t num_pages, float* keys, float* values,
                               void* stream) {
    return sfg_hip_kv_gather_pool_v1(k_pool, v_pool, SFG_BF16, page_table, batch, kv_heads, length,
                                     head_dim, page_tokens, pages_per_seq, num_pages, keys, values,
                                     stream);
}

size_t sfg_hip_moe_route_workspace_v1(int64_t tokens, int64_t experts, int64_t top_k) {
    return sfg::moe_route_workspace_bytes(tokens, experts, top_k);
}

int sfg_hip_moe_route_v1(const float* x, const float* router, const float* bias, int64_t tokens,
                         int64_t hidden, int64_t experts, int64_t top_k, int32_t* ids,
                         float* weights, int32_t* counts, int32_t* offsets, int32_t* token_ids,
                         int32_t* route_slots, float* routing_weights, int32_t* position,
                         void* workspace, size_t workspace_bytes, void* stream) {
    (void)workspace; (void)workspace_bytes;
    // validate_config (moe_compiler.cpp:41-45)
    if (!x || !router || !ids || !weights || !counts || !offsets || !token_ids || !route_slots ||
        !routing_weights || !position || tokens <= 0 || hidden <= 0 || experts <= 0 ||
        top_k <= 0 || top_k > experts)
        return fail(SFG_ERR_INVALID_CONFIG, "invalid MoE configuration");
    int rc = sfg::launch_moe_router(x, router, bias, tokens, hidden, experts, top_k, ids, weights,
                                    as_stream(stream));
    if (rc != SFG_OK) return fail(rc, "moe_route: experts %lld / top_k %lld not lowered",
                                  (long long)experts, (long long)top_k);
    rc = sfg::launch_moe_dispatch(ids, weights, tokens, experts, top_k, counts, offsets, token_ids,
                                  route_slots, routing_weights, position, as_stream(stream));
    if (rc != SFG_OK) return fail(rc, "moe_dispatch: not lowered");
    return check_launch("moe_route");
}

int sfg_hip_moe_dispatch_trace_v1(const int32_t* ids, const float* weights, int64_t tokens,
                                  int64_t experts, int64_t top_k, int32_t* counts,
                                  int32_t* offsets, int32_t* token_ids, int32_t* route_slots,
                                  float* routing_weights, int32_t* position, void* stream) {
    if (!ids || !weights || !counts || !offsets || !token_ids || !route_slots ||
        !routing_weights || !position || tokens <= 0 || experts <= 0 || top_k <= 0 ||
        top_k > experts)
        return fail(SFG_ERR_INVALID_CONFIG, "routing trace does not match MoE configuration");
    const int rc = sfg::launch_moe_dispatch(ids, weights, tokens, experts, top_k, counts, offsets,
                                            token_ids, route_slots, routing_weights, position,
                                            as_stream(stream));
    if (rc != SFG_OK) return fail(rc, "moe_dispatch: not lowered");
    return check_launch("moe_dispatch_trace");
}

size_t sfg_hip_moe_expert_workspace_v1(int64_t tokens, int64_t hidden, int64_t inter,
                                       int64_t experts, int64_t top_k) {
    (void)tokens; (void)hidden; (void)inter; (void)experts; (void)top_k;
    return 0;
}

// The grouped expert products of execute_moe (moe_compiler.cpp:64-155): x and
// act in the activation dtype (bf16, or fp32 with fp32 weights).
static int moe_experts(const void* x, int act_dtype, const int32_t* offsets, const int32_t* token_ids,
                       const void* w13, const float* s13, const void* w2, const float* s2,
                       int w_dtype, int w_layout, void* act, float* y, int64_t tokens, int64_t hidden,
                       int64_t inter, int64_t experts, int64_t top_k, int tile, hipStream_t stream) {
    sfg::GemmProblem p{};
    p.a = x; p.a_dtype = act_dtype; p.lda = hidden; p.a_rows = token_ids; p.a_rows_limit = tokens;
    p.b = w13; p.b_dtype = w_dtype; p.ldb = hidden; p.b_scales = s13;
    p.b_group_stride = 2 * inter * hidden; p.s_group_stride = 2 * inter;
    p.c = act; p.c_dtype = act_dtype; p.ldc = inter;
    p.m = tokens * top_k; p.n = inter; p.k = hidden; p.epilogue = SFG_EPI_GLU_SILU_UP;
    p.b_layout = w_layout;
    p.offsets = offsets; p.groups = static_cast<int>(experts);
    p.tile = tile;
    int rc = sfg::launch_gemm(p, nullptr, 0, stream);
    if (rc != SFG_OK) return fail(rc, "moe experts W1/W3: shape not lowered (H=%lld I=%lld)",
                                  (long long)hidden, (long long)inter);
    sfg::GemmProblem q{};
    q.a = act; q.a_dtype = act_dtype; q.lda = inter; q.a_rows = nullptr;
    q.b = w2; q.b_dtype = w_dtype; q.ldb = inter; q.b_scales = s2;
    q.b_group_stride = hidden * inter; q.s_group_stride = hidden;
    q.c = y; q.c_dtype = SFG_F32; q.ldc = hidden;
    q.m = tokens * top_k; q.n = hidden; q.k = inter; q.epilogue = SFG_EPI_NONE;
    q.b_layout = w_layout;
    q.offsets = offsets; q.groups = static_cast<int>(experts);
    q.tile = tile;
    rc = sfg::launch_gemm(q, nullptr, 0, stream);
    if (rc != SFG_OK) return fail(rc, "moe experts W2: shape not lowered");
    return check_launch("moe_experts");
}

int sfg_hip_moe_experts_v1(const uint16_t* x, const int32_t* offsets, const int32_t* token_ids,
                           const void* w13, const float* s13, const void* w2, const float* s2,
                           int w_dtype, int w_layout, uint16_t* act, float* y, int64_t tokens, int64_t hidden,
                           int64_t inter, int64_t experts, int64_t top_k, void* workspace,
                           size_t workspace_bytes, void* stream) {
    (void)workspace; (void)workspace_bytes;
    if (!x || !offsets || !token_ids || !w13 || !w2 || !act || !y || tokens <= 0 || hidden <= 0 ||
        inter <= 0 || experts <= 0 || top_k <= 0 || top_k > experts)
        return fail(SFG_ERR_INVALID_CONFIG, "invalid MoE configuration");
    if (w_dtype == SFG_I8 && (!s13 || !s2)) return fail(SFG_ERR_SHAPE, "int8 experts need scales");
    if (w_dtype != SFG_BF16 && w_dtype != SFG_I8) return fail(SFG_ERR_UNSUPPORTED, "expert dtype %d", w_dtype);
    if (w_layout != SFG_LAYOUT_NK && w_layout != SFG_LAYOUT_TILED)
        return fail(SFG_ERR_SHAPE, "moe experts: unknown weight layout %d", w_layout);
    return moe_experts(x, SFG_BF16, offsets, token_ids, w13, s13, w2, s2, w_dtype, w_layout, act, y,
                       tokens, hidden, inter, experts, top_k, SFG_TILE_AUTO, as_stream(stream));
}

int sfg_hip_moe_combine_v1(const float* y, const int32_t* position, const float* weights,
                           const float* residual, float* out, int64_t tokens, int64_t hidden,
                           int64_t top_k, void* stream) {
    if (!y || !position || !weights || !residual || !out || tokens <= 0 || hidden <= 0 || top_k <= 0)
        return fail(SFG_ERR_SHAPE, "moe_combine: invalid arguments");
    sfg::launch_moe_combine(y, position, weights, residual, out, tokens, hidden, top_k,
                            as_stream(stream));
    return check_launch("moe_combine");
}

// ---------------------------------------------------------------------------
// Whole layer.
// ---------------------------------------------------------------------------

}  // extern "C"

namespace {

struct LayerBuffers {
    void* xn = nullptr;       // [rows][H] act dtype
    float* xn2_f32 = nullptr; // MoE router input [rows][H]
    float* qkv = nullptr;     // [rows][qkvw]
    void* q = nullptr;        // prefill: [B][Hq][S][D] act; decode: fp32 [B][Hq][D]
    void* k = nullptr;
    void* v = nullptr;
    void* attn = nullptr;     // merged [rows][H] act dtype
    float* r1 = nullptr;      // [rows][H]
    void* act = nullptr;      // dense [rows][I] / MoE [rows*k][I]
    float* y = nullptr;       // MoE [rows*k][H]
    int32_t* ids = nullptr; float* wts = nullptr; int32_t* counts = nullptr;
    int32_t* offsets = nullptr; int32_t* token_ids = nullptr; int32_t* slots = nullptr;
    float* rweights = nullptr; int32_t* position = nullptr;
    void* attn_ws = nullptr;
    void* gemm_ws = nullptr; size_t gemm_ws_bytes = 0;
    size_t total = 0;
};

int validate_desc(const sfg_layer_desc* d) {
    if (!d) return fail(SFG_ERR_INVALID_CONFIG, "null layer descriptor");
    if (d->abi != SFG_HIP_ABI_VERSION)
        return fail(SFG_ERR_ABI, "layer descriptor ABI %d, library ABI %d", d->abi, SFG_HIP_ABI_VERSION);
    // validate (decoder_compiler.cpp:26-39)
    if (d->batch <= 0 || d->sequence <= 0 || d->hidden <= 0 || d->intermediate <= 0 ||
        d->query_heads <= 0 || d->kv_heads <= 0 || d->head_dim <= 0 ||
        d->hidden != d->query_heads * d->head_dim || d->query_heads % d->kv_heads != 0 ||
        !(d->rms_epsilon > 0.0f))
        return fail(SFG_ERR_INVALID_CONFIG, "invalid decoder configuration");
    if (d->ffn == 1 && (d->experts <= 0 || d->top_k <= 0 || d->top_k > d->experts))
        return fail(SFG_ERR_INVALID_CONFIG, "invalid decoder MoE configuration");
    if (d->context < 0) return fail(SFG_ERR_INVALID_CONFIG, "invalid decoder context sequence");
    if (d->act_dtype != SFG_F32 && d->act_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "activation dtype %d", d->act_dtype);
    if (d->act_dtype == SFG_F32 && d->weight_dtype != SFG_F32)
        return fail(SFG_ERR_UNSUPPORTED, "fp32 activations need fp32 weights");
    if (d->act_dtype == SFG_BF16 && d->weight_dtype != SFG_BF16 && d->weight_dtype != SFG_I8)
        return fail(SFG_ERR_UNSUPPORTED, "bf16 activations need bf16 or int8 weights");
    if (d->head_dim > 256)
        return fail(SFG_ERR_UNSUPPORTED, "head_dim %d: attention lowers head dims up to 256", d->head_dim);
    if (d->context > 0) {
        // the paged pools hold the activation dtype: fp32 for the fp32 path, bf16 otherwise
        if (d->page_tokens <= 0 || d->pages_per_seq <= 0 || d->num_pages <= 0)
            return fail(SFG_ERR_INVALID_CONFIG, "invalid paged KV configuration");
        if (d->context > d->pages_per_seq * d->page_tokens)
            return fail(SFG_ERR_GUARD, "KV cache length violates compiled guard");
        // validate_config (attention_compiler.cpp:23-29): the step's causal
        // query block attends over the cached keys
        if (d->causal && !d->kv_append && d->sequence > d->context)
            return fail(SFG_ERR_INVALID_CONFIG, "invalid attention configuration");
        if (d->kv_append && d->context + d->sequence > d->pages_per_seq * d->page_tokens)
            return fail(SFG_ERR_GUARD, "paged KV capacity exceeded by the appended tokens");
    } else if (d->kv_append) {
        return fail(SFG_ERR_INVALID_CONFIG, "kv append needs a decode step (context > 0)");
    }
    if (d->weight_layout != SFG_LAYOUT_NK && d->weight_layout != SFG_LAYOUT_TILED)
        return fail(SFG_ERR_SHAPE, "unknown weight layout %d", d->weight_layout);
    if (d->gemm_tile < SFG_TILE_AUTO || d->gemm_tile >= SFG_TILE_COUNT)
        return fail(SFG_ERR_SHAPE, "unknown GEMM tile policy %d", d->gemm_tile);
    if (d->attn_waves != 0 && d->attn_waves != 4 && d->attn_waves != 8)
        return fail(SFG_ERR_SHAPE, "flash prefill waves %d (0, 4 or 8)", d->attn_waves);
    if (d->weight_layout == SFG_LAYOUT_TILED && d->act_dtype != SFG_BF16)
        return fail(SFG_ERR_UNSUPPORTED, "tiled weights are bf16 / int8");
    return SFG_OK;
}

// The decode attention of a layer step: the keys it may reach (the cache,
// plus the step's own tokens when they are appended) and the kernel choice.
DecodePlan layer_decode_plan(const sfg_layer_desc* d) {
    const int64_t keys = static_cast<int64_t>(d->context) + (d->kv_append ? d->sequence : 0);
    return plan_decode(d->act_dtype, d->batch, d->query_heads, d->kv_heads, d->sequence, d->head_dim,
                       d->page_tokens, keys, d->kv_splits);
}

// The flash prefill over V^T serves bf16 activations at head_dim 128.
bool use_vt(const sfg_layer_desc* d) {
    return d->context == 0 && d->act_dtype == SFG_BF16 && d->head_dim == 128;
}

LayerBuffers plan_buffers(const sfg_layer_desc* d, void* ws) {
    LayerBuffers b;
    Carve c(ws);
    const int64_t rows = static_cast<int64_t>(d->batch) * d->sequence;
    const int64_t H = d->hidden, I = d->intermediate, D = d->head_dim;
    const int64_t kvd = static_cast<int64_t>(d->kv_heads) * D;
    const int64_t qkvw = H + 2 * kvd;
    const size_t ae = d->act_dtype == SFG_F32 ? 4 : 2;
    const bool moe = d->ffn == 1;
    b.xn = c.take(rows * H * ae);
    if (moe) b.xn2_f32 = static_cast<float*>(c.take(rows * H * 4));
    b.qkv = static_cast<float*>(c.take(rows * qkvw * 4));
    if (d->context == 0) {
        b.q = c.take(rows * H * ae);
        b.k = c.take(rows * kvd * ae);
        // bf16 head_dim-128 prefill keeps V transposed, keys padded to 64
        b.v = use_vt(d) ? c.take(static_cast<int64_t>(d->batch) * kvd *
                                 sfg::attn_vt_ld(d->sequence) * 2)
                        : c.take(rows * kvd * ae);
    }
    b.attn = c.take(rows * H * ae);
    b.r1 = static_cast<float*>(c.take(rows * H * 4));
    if (moe) {
        const int64_t assign = rows * d->top_k;
        b.act = c.take(assign * I * ae);
        b.y = static_cast<float*>(c.take(assign * H * 4));
        b.ids = static_cast<int32_t*>(c.take(assign * 4));
        b.wts = static_cast<float*>(c.take(assign * 4));
        b.counts = static_cast<int32_t*>(c.take(static_cast<size_t>(d->experts) * 4));
        b.offsets = static_cast<int32_t*>(c.take(static_cast<size_t>(d->experts + 1) * 4));
        b.token_ids = static_cast<int32_t*>(c.take(assign * 4));
        b.slots = static_cast<int32_t*>(c.take(assign * 4));
        b.rweights = static_cast<float*>(c.take(assign * 4));
        b.position = static_cast<int32_t*>(c.take(assign * 4));
    } else {
        b.act = c.take(rows * I * ae);
    }
    if (d->context > 0) b.attn_ws = c.take(layer_decode_plan(d).bytes);
    // Split-K scratch sized for the widest projection.
    size_t g = 0;
    const int64_t ns[4] = {qkvw, H, 2 * I, H};
    const int64_t ks[4] = {H, H, H, I};
    for (int i = 0; i < 4; ++i) {
        const size_t s = sfg::gemm_workspace_bytes(rows, ns[i], ks[i]);
        if (s > g) g = s;
    }
    b.gemm_ws_bytes = g;
    b.gemm_ws = c.take(g);
    b.total = c.used;
    return b;
}

struct Marks {
    void** ev;
    hipStream_t s;
    void mark(int id) const {
        if (ev && ev[id]) (void)hipEventRecord(static_cast<hipEvent_t>(ev[id]), s);
    }
};

}  // namespace

extern "C" {

size_t sfg_hip_decoder_layer_workspace_v1(const sfg_layer_desc* desc) {
    if (validate_desc(desc) != SFG_OK) return 0;
    return plan_buffers(desc, nullptr).total;
}

int sfg_hip_decoder_layer_tap_v1(const sfg_layer_desc* d, int tap, size_t* offset, size_t* bytes,
                                 int* dtype) {
    int rc = validate_desc(d);
    if (rc != SFG_OK) return rc;
    if (!offset || !bytes || !dtype) return fail(SFG_ERR_SHAPE, "decoder layer tap: null output");
    // Offsets are the carve-up of a workspace based at a non-null sentinel.
    char* const base = reinterpret_cast<char*>(static_cast<uintptr_t>(1) << 20);
    const LayerBuffers b = plan_buffers(d, base);
    const int64_t rows = static_cast<int64_t>(d->batch) * d->sequence;
    const int64_t H = d->hidden;
    const bool routed = d->ffn == 1 && !d->use_routing_trace;
    const void* p = nullptr;
    size_t n = 0;
    int dt = SFG_F32;
    switch (tap) {
    case SFG_TAP_ATTN:
        p = b.attn; dt = d->act_dtype; n = static_cast<size_t>(rows * H) * (dt == SFG_F32 ? 4 : 2);
        break;
    case SFG_TAP_RESIDUAL1:
        p = b.r1; n = static_cast<size_t>(rows * H) * 4;
        break;
    case SFG_TAP_NORM2:
        p = b.xn; dt = d->act_dtype; n = static_cast<size_t>(rows * H) * (dt == SFG_F32 ? 4 : 2);
        break;
    case SFG_TAP_ROUTE_INPUT:
        if (d->ffn != 1) return fail(SFG_ERR_UNSUPPORTED, "the router input tap needs a MoE layer");
        p = b.xn2_f32; n = static_cast<size_t>(rows * H) * 4;
        break;
    case SFG_TAP_ROUTE_IDS:
    case SFG_TAP_ROUTE_WEIGHTS:
        if (!routed) return fail(SFG_ERR_UNSUPPORTED, "routing taps need a MoE layer routed on the device");
        p = tap == SFG_TAP_ROUTE_IDS ? static_cast<const void*>(b.ids) : static_cast<const void*>(b.wts);
        dt = tap == SFG_TAP_ROUTE_IDS ? SFG_I32 : SFG_F32;
        n = static_cast<size_t>(rows * d->top_k) * 4;
        break;
    default:
        return fail(SFG_ERR_SHAPE, "unknown decoder layer tap %d", tap);
    }
    *offset = static_cast<size_t>(static_cast<const char*>(p) - base);
    *bytes = n;
    *dtype = dt;
    return SFG_OK;
}

int sfg_hip_decoder_layer_v1(const sfg_layer_desc* d, const sfg_layer_weights* w,
                             const sfg_layer_io* io, void* workspace, size_t workspace_bytes,
                             void* stream_ptr) {
    int rc = validate_desc(d);
    if (rc != SFG_OK) return rc;
    if (!w || !io || !io->x || !io->out) return fail(SFG_ERR_SHAPE, "decoder layer: null weights or io");
    const hipStream_t s = as_stream(stream_ptr);
    const LayerBuffers need = plan_buffers(d, nullptr);
    if (!workspace || workspace_bytes < need.total)
        return fail(SFG_ERR_WORKSPACE, "decoder layer: workspace %zu < %zu", workspace_bytes, need.total);
    const LayerBuffers b = plan_buffers(d, workspace);
    const bool moe = d->ffn == 1;
    const bool decode = d->context > 0;
    const int64_t rows = static_cast<int64_t>(d->batch) * d->sequence;
    const int64_t H = d->hidden, I = d->intermediate, D = d->head_dim;
    const int64_t kvd = static_cast<int64_t>(d->kv_heads) * D;
    const int64_t qkvw = H + 2 * kvd;
    const int act = d->act_dtype;
    const int wdt = d->weight_dtype;
    if (!w->rms1 || !w->rms2 || !w->w_qkv || !w->w_o || (!w->rope_table && D >= 2))
        return fail(SFG_ERR_SHAPE, "decoder layer: missing attention weights");
    if (wdt == SFG_I8 && (!w->s_qkv || !w->s_o)) return fail(SFG_ERR_SHAPE, "int8 weights need scales");
    if (moe) {
        if (!w->router || !w->w13 || !w->w2) return fail(SFG_ERR_SHAPE, "MoE layer: missing expert weights");
        if (wdt == SFG_I8 && (!w->s13 || !w->s2)) return fail(SFG_ERR_SHAPE, "int8 experts need scales");
        if (d->use_routing_trace && (!io->trace_ids || !io->trace_weights))
            return fail(SFG_ERR_SHAPE, "routing trace requested but not supplied");
    } else {
        if (!w->w_gate_up || !w->w_down) return fail(SFG_ERR_SHAPE, "dense layer: missing FFN weights");
        if (wdt == SFG_I8 && (!w->s_gate_up || !w->s_down)) return fail(SFG_ERR_SHAPE, "int8 weights need scales");
    }
    if (decode && (!w->k_pool || !w->v_pool || !w->page_table))
        return fail(SFG_ERR_SHAPE, "decode step needs the paged KV pools and page table");

    const Marks mk{io->stage_events, s};
    auto gemm = [&](const void* a, int64_t lda, const void* bw, const float* bs, void* c, int c_dtype,
                    const float* res, int64_t m, int64_t n, int64_t k, int epi, int64_t ldc = 0) -> int {
        sfg::GemmProblem p{};
        p.a = a; p.a_dtype = act; p.lda = lda;
        p.b = bw; p.b_dtype = wdt; p.ldb = k; p.b_scales = bs;
        p.c = c; p.c_dtype = c_dtype; p.ldc = ldc > 0 ? ldc : n;
        p.residual = res; p.ldr = n;
        p.m = m; p.n = n; p.k = k; p.epilogue = epi; p.groups = 1;
        p.b_layout = d->weight_layout;
        p.tile = d->gemm_tile;
        const int r = sfg::launch_gemm(p, b.gemm_ws, b.gemm_ws_bytes, s);
        if (r != SFG_OK)
            return fail(r, "decoder layer GEMM %lldx%lldx%lld not lowered for dtype %d/%d",
                        (long long)m, (long long)n, (long long)k, act, wdt);
        return SFG_OK;
    };

    mk.mark(SFG_MARK_START);
    // 1. RMSNorm
    sfg::launch_rmsnorm(io->x, w->rms1, b.xn, act, rows, H, d->rms_epsilon, s);
    mk.mark(SFG_MARK_NORM1);
    // 2. fused QKV projection -> fp32
    const float scale = default_scale(D, 0.0f);
    const bool vt = use_vt(d);
    const int64_t ld_vt = vt ? sfg::attn_vt_ld(d->sequence) : 0;
    // bf16 prefill: the QKV GEMM's epilogue writes the RoPE'd Q / K and V^T
    // itself (split_qkv + apply_rope, decoder_compiler.cpp:96-148) when the
    // direct-to-LDS path takes the shape; otherwise the product goes to fp32
    // rows and the split + RoPE kernels follow.
    sfg::GemmProblem qp{};
    qp.a = b.xn; qp.a_dtype = act; qp.lda = H;
    qp.b = w->w_qkv; qp.b_dtype = wdt; qp.ldb = H; qp.b_scales = w->s_qkv;
    qp.m = rows; qp.n = qkvw; qp.k = H; qp.epilogue = sfg::kEpiQkvRope; qp.groups = 1;
    qp.b_layout = d->weight_layout;
    qp.tile = d->gemm_tile;
    qp.qkv = sfg::QkvRopeOut{reinterpret_cast<const float2*>(w->rope_table), d->sequence, d->query_heads,
                             d->kv_heads, static_cast<uint16_t*>(b.q), static_cast<uint16_t*>(b.k),
                             static_cast<uint16_t*>(b.v), ld_vt};
    const bool fused_qkv = vt && !decode && sfg::gemm_qkv_rope_supported(qp);
    if (fused_qkv) {
        if (ld_vt != d->sequence) sfg::launch_fill_zero(b.v, static_cast<size_t>(d->batch) * kvd * ld_vt * 2, s);
        const int r = sfg::launch_gemm(qp, b.gemm_ws, b.gemm_ws_bytes, s);
        if (r != SFG_OK) return fail(r, "decoder layer QKV GEMM with RoPE epilogue not lowered");
    } else if ((rc = gemm(b.xn, H, w->w_qkv, w->s_qkv, b.qkv, SFG_F32, nullptr, rows,
                          // a reference decode step attends over the cache only and
                          // discards the step's K / V (decoder_compiler.cpp:238-243):
                          // only the Q columns are computed (the first H weight rows,
                          // a prefix in both weight layouts), into the same rows
                          decode && !d->kv_append ? H : qkvw, H, SFG_EPI_NONE, qkvw))) {
        return rc;
    }
    mk.mark(SFG_MARK_QKV);
    // 3. split + RoPE (decode keeps only Q: the step's K/V are discarded,
    //    decoder_compiler.cpp:238-243)
    if (!decode && !fused_qkv) {
        sfg::launch_split_rope(b.qkv, w->rope_table, d->batch, d->sequence, d->query_heads,
                               d->kv_heads, D, b.q, b.k, vt ? nullptr : b.v, act, s);
        if (vt)
            sfg::launch_v_transpose(b.qkv, d->batch, d->sequence, d->query_heads, d->kv_heads, ld_vt,
                                    static_cast<uint16_t*>(b.v), s);
    }
    mk.mark(SFG_MARK_ROPE);
    // 4. attention -> merged [rows][H]
    if (decode) {
        const bool append = d->kv_append != 0;
        const int64_t S = d->sequence;
        const int64_t capacity = static_cast<int64_t>(d->pages_per_seq) * d->page_tokens;
        const DecodePlan plan = layer_decode_plan(d);
        if (append) {
            // Append mode: the step's K (rotated at its true positions, the
            // sequence's length onwards) and V go into the pools there, as
            // append_paged_kv does (next_milestones.cpp:486-524).  Row (b, t)
            // of the QKV product is b S + t.
            rc = sfg::launch_kv_append(b.qkv + H, b.qkv + H + kvd, SFG_F32, S * qkvw, D, qkvw,
                                       w->rope_table, w->k_pool, w->v_pool, act, w->page_table,
                                       io->seq_lens, d->context, 0, d->batch, d->kv_heads, S, D,
                                       d->page_tokens, d->pages_per_seq, d->num_pages, s);
            if (rc != SFG_OK) return fail(rc, "kv append not lowered (head_dim %lld)", (long long)D);
        }
        // RoPE of the step's queries is applied while the kernel loads Q
        // straight from the QKV rows: at the index within the step, as the
        // reference rotates it (decoder_compiler.cpp:96-104), or in append mode
        // at the true positions, over the cache including the new tokens.
        hipEvent_t mid = io->stage_events ? static_cast<hipEvent_t>(io->stage_events[SFG_MARK_ATTN_MAIN]) : nullptr;
        if (plan.mfma) {
            rc = sfg::launch_attn_decode_paged(
                b.qkv, qkvw, w->rope_table, append ? -1 : 0, static_cast<const uint16_t*>(w->k_pool),
                static_cast<const uint16_t*>(w->v_pool), w->page_table, append ? io->seq_lens : nullptr,
                d->context, append ? 1 : 0, b.attn, act, d->batch, d->query_heads, d->kv_heads, D,
                d->page_tokens, d->pages_per_seq, d->num_pages, plan.splits, scale, b.attn_ws, s, mid);
        } else {
            // any head_dim / page size / step length / pool dtype: query row i
            // of a sequence sees key j <= keys - S + i (attention_compiler.cpp:68-72)
            sfg::PagedRowsLaunch a{};
            a.q = b.qkv; a.q_stride_b = S * qkvw; a.q_stride_i = qkvw; a.q_stride_h = D;
            a.rope = w->rope_table; a.rope_rows = static_cast<int>(append ? capacity : S);
            a.rope_pos = append ? -1 : 0;
            a.k_pool = w->k_pool; a.v_pool = w->v_pool; a.kv_dtype = act;
            a.page_table = w->page_table; a.seq_lens = append ? io->seq_lens : nullptr;
            a.max_context = d->context; a.len_extra = append ? static_cast<int>(S) : 0;
            a.out = b.attn; a.out_dtype = act;
            a.out_stride_b = S * H; a.out_stride_i = H; a.out_stride_h = D;
            a.batch = d->batch; a.q_heads = d->query_heads; a.kv_heads = d->kv_heads; a.seq_q = S;
            a.head_dim = D; a.page_tokens = d->page_tokens; a.pages_per_seq = d->pages_per_seq;
            a.num_pages = d->num_pages; a.splits = plan.splits; a.causal = d->causal; a.scale = scale;
            a.mid_event = mid;
            rc = sfg::launch_attn_paged_rows(a, b.attn_ws, s);
        }
        if (rc != SFG_OK) return fail(rc, "decode attention not lowered (head_dim %lld)", (long long)D);
        if (append && io->seq_lens) sfg::launch_kv_advance(io->seq_lens, d->batch, S, capacity, s);
    } else {
        if (act == SFG_F32) {
            rc = sfg::launch_attn_prefill_f32(static_cast<const float*>(b.q), static_cast<const float*>(b.k),
                                              static_cast<const float*>(b.v), b.attn, act, d->batch,
                                              d->query_heads, d->kv_heads, d->sequence, d->sequence, D,
                                              d->causal, scale, s);
            if (rc != SFG_OK) return fail(rc, "fp32 attention head_dim %lld not lowered", (long long)D);
        } else if (vt) {
            rc = sfg::launch_attn_prefill_vt(static_cast<const uint16_t*>(b.q),
                                             static_cast<const uint16_t*>(b.k),
                                             static_cast<const uint16_t*>(b.v), ld_vt, b.attn, act,
                                             d->batch, d->query_heads, d->kv_heads, d->sequence,
                                             d->sequence, D, d->causal, scale, d->attn_waves, s);
            if (rc != SFG_OK) return fail(rc, "bf16 prefill attention not lowered (head_dim %lld)", (long long)D);
        } else {
            rc = sfg::launch_attn_prefill_bf16(static_cast<const uint16_t*>(b.q),
                                               static_cast<const uint16_t*>(b.k),
                                               static_cast<const uint16_t*>(b.v), b.attn, act,
                                               d->batch, d->query_heads, d->kv_heads, d->sequence,
                                               d->sequence, D, d->causal, scale, s);
            if (rc != SFG_OK) return fail(rc, "bf16 prefill attention not lowered (head_dim %lld)", (long long)D);
        }
        mk.mark(SFG_MARK_ATTN_MAIN);
    }
    mk.mark(SFG_MARK_ATTN);
    // 5. O-projection + residual: r1 = attn Wo + x
    if ((rc = gemm(b.attn, H, w->w_o, w->s_o, b.r1, SFG_F32, io->x, rows, H, H, SFG_EPI_RESIDUAL)))
        return rc;
    mk.mark(SFG_MARK_OPROJ);
    // 6. RMSNorm
    // (MoE: the router reads the same rows in fp32, written by the same pass)
    sfg::launch_rmsnorm(b.r1, w->rms2, b.xn, act, rows, H, d->rms_epsilon, s, moe ? b.xn2_f32 : nullptr);
    mk.mark(SFG_MARK_NORM2);
    if (!moe) {
        mk.mark(SFG_MARK_ROUTE);
        // 7. gate_up + SwiGLU -> act ; down + residual -> out
        if ((rc = gemm(b.xn, H, w->w_gate_up, w->s_gate_up, b.act, act, nullptr, rows, I, H, SFG_EPI_SWIGLU)))
            return rc;
        mk.mark(SFG_MARK_FFN_UP);
        if ((rc = gemm(b.act, I, w->w_down, w->s_down, io->out, SFG_F32, b.r1, rows, H, I, SFG_EPI_RESIDUAL)))
            return rc;
        mk.mark(SFG_MARK_FFN_DOWN);
    } else {
        const int64_t E = d->experts, K = d->top_k;
        if (d->use_routing_trace) {
            rc = sfg::launch_moe_dispatch(io->trace_ids, io->trace_weights, rows, E, K, b.counts,
                                          b.offsets, b.token_ids, b.slots, b.rweights, b.position, s);
        } else {
            rc = sfg::launch_moe_router(b.xn2_f32, w->router, w->router_bias, rows, H, E, K, b.ids,
                                        b.wts, s);
            if (rc != SFG_OK) return fail(rc, "MoE router not lowered (E=%lld k=%lld)", (long long)E, (long long)K);
            rc = sfg::launch_moe_dispatch(b.ids, b.wts, rows, E, K, b.counts, b.offsets, b.token_ids,
                                          b.slots, b.rweights, b.position, s);
        }
        if (rc != SFG_OK) return fail(rc, "MoE dispatch not lowered");
        mk.mark(SFG_MARK_ROUTE);
        const float* route_w = d->use_routing_trace ? io->trace_weights : b.wts;
        rc = moe_experts(b.xn, act, b.offsets, b.token_ids, w->w13, w->s13, w->w2, w->s2, wdt,
                         d->weight_layout, b.act, b.y, rows, H, I, E, K, d->gemm_tile, s);
        if (rc != SFG_OK) return rc;
        mk.mark(SFG_MARK_FFN_UP);
        sfg::launch_moe_combine(b.y, b.position, route_w, b.r1, io->out, rows, H, K, s);
        mk.mark(SFG_MARK_FFN_DOWN);
    }
    mk.mark(SFG_MARK_END);
    return check_launch("decoder_layer");
}

int sfg_hip_events_create_v1(int count, void** events) {
    if (count <= 0 || !events) return fail(SFG_ERR_SHAPE, "events_create: invalid");
    for (int i = 0; i < count; ++i) {
        hipEvent_t e;
        const hipError_t r = hipEventCreate(&e);
        if (r != hipSuccess) return fail(SFG_ERR_DEVICE, "hipEventCreate: %s", hipGetErrorString(r));
        events[i] = e;
    }
    return SFG_OK;
}

int sfg_hip_events_destroy_v1(int count, void** events) {
    if (count < 0 || (count > 0 && !events)) return fail(SFG_ERR_SHAPE, "events_destroy: invalid");
    for (int i = 0; i < count; ++i)
        if (events[i]) (void)hipEventDestroy(static_cast<hipEvent_t>(events[i]));
    return SFG_OK;
}

int sfg_hip_event_elapsed_v1(void* start, void* end, float* ms) {
    if (!start || !end || !ms) return fail(SFG_ERR_SHAPE, "event_elapsed: invalid");
    const hipError_t r = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end));
    if (r != hipSuccess) return fail(SFG_ERR_DEVICE, "hipEventElapsedTime: %s", hipGetErrorString(r));
    return SFG_OK;
}

int sfg_hip_stream_synchronize_v1(void* stream) {
    const hipError_t r = hipStreamSynchronize(as_stream(stream));
    if (r != hipSuccess) return fail(SFG_ERR_DEVICE, "hipStreamSynchronize: %s", hipGetErrorString(r));
    return SFG_OK;
}

}  // extern "C"
