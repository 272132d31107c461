// C++20 host runtime over libsfg_hip.so: DecoderCompiler::compile and
// execute_decoder_layer for gfx950 plans.  Reference behaviour followed:
//   compile            decoder_compiler.cpp:518-620 (validate, pack constants
//                      once, plan memory); concatenate_columns 77-94
//   execute_once       decoder_compiler.cpp:218-304 (one sfg_hip_decoder_layer_v1)
//   execute_decoder_layer decoder_compiler.cpp:675-692 (warmup, median, tokens/s)
//   library loading    aot_runtime.cpp:152-196, 259 (dlopen, dlsym, metadata check)
//   paged KV           next_milestones.cpp:29-33, 472-581 (page -> physical slot)
#include "sfg_decoder.hpp"
#include "sfg_runtime_internal.hpp"

#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <thread>

namespace schedforge::hip {
namespace {


// libsfg_hip.so beside the library (or executable) that holds this code.
std::filesystem::path default_library_path() {
    if (const char* env = std::getenv("SFG_HIP_LIBRARY"); env && *env) return env;
    Dl_info info{};
    if (dladdr(reinterpret_cast<void*>(&default_library_path), &info) && info.dli_fname) {
        const auto here = std::filesystem::absolute(info.dli_fname).parent_path();
        for (const auto& candidate : {here / "libsfg_hip.so", here / ".." / "lib" / "libsfg_hip.so"})
            if (std::filesystem::exists(candidate)) return candidate;
    }
    throw std::runtime_error("libsfg_hip.so not found (set SFG_HIP_LIBRARY or build the package)");
}


// ---------------------------------------------------------------- numerics

// fp32 -> bf16 bits by round to nearest even, no NaN special case
// (convert_to_bf16, compiler.cpp:34-43).
std::uint16_t bf16_bits(float value) {
    std::uint32_t bits;
    std::memcpy(&bits, &value, sizeof bits);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return static_cast<std::uint16_t>(bits >> 16);
}

unsigned worker_count() {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    return std::min(hw, 16u);
}

// Runs body(begin, end) over [0, count) on up to worker_count() threads.
template <typename Body>
void parallel_for(std::int64_t count, Body body) {
    const std::int64_t workers = std::min<std::int64_t>(worker_count(), std::max<std::int64_t>(1, count / 65536));
    if (workers <= 1) {
        body(0, count);
        return;
    }
    std::vector<std::thread> threads;
    const std::int64_t chunk = (count + workers - 1) / workers;
    for (std::int64_t w = 0; w < workers; ++w) {
        const std::int64_t begin = w * chunk, end = std::min(count, begin + chunk);
        if (begin < end) threads.emplace_back([=] { body(begin, end); });
    }
    for (auto& t : threads) t.join();
}

// Element i: Box-Muller (cosine branch) in double on two 53-bit uniforms drawn
// from the counter stream at 2i and 2i+1.
std::vector<float> normal(std::uint64_t seed, std::uint32_t tensor_id, std::size_t count,
                          float stddev) {
    std::vector<float> out(count);
    const std::uint64_t key = stream_key(seed, tensor_id);
    constexpr double two_pi = 6.283185307179586476925286766559;
    parallel_for(static_cast<std::int64_t>(count), [&](std::int64_t begin, std::int64_t end) {
        for (std::int64_t i = begin; i < end; ++i) {
            const std::uint64_t r1 = splitmix64(key + 2 * static_cast<std::uint64_t>(i));
            const std::uint64_t r2 = splitmix64(key + 2 * static_cast<std::uint64_t>(i) + 1);
            const double u1 = (static_cast<double>(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
            const double u2 = static_cast<double>(r2 >> 11) * (1.0 / 9007199254740992.0);
            const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
            out[i] = static_cast<float>(static_cast<double>(stddev) * z);
        }
    });
    return out;
}

std::vector<std::int32_t> page_permutation(std::uint64_t seed, std::int64_t count) {
    std::vector<std::int32_t> perm(count);
    for (std::int64_t i = 0; i < count; ++i) perm[i] = static_cast<std::int32_t>(i);
    const std::uint64_t key = stream_key(seed, 17u);
    for (std::int64_t i = count - 1; i > 0; --i) {
        const std::uint64_t r = splitmix64(key + static_cast<std::uint64_t>(i));
        std::swap(perm[i], perm[static_cast<std::int64_t>(r % static_cast<std::uint64_t>(i + 1))]);
    }
    return perm;
}

void round_in_place(std::vector<float>& values) {
    parallel_for(static_cast<std::int64_t>(values.size()), [&](std::int64_t begin, std::int64_t end) {
        for (std::int64_t i = begin; i < end; ++i) values[i] = round_to_bf16(values[i]);
    });
}

void require_size(const std::vector<float>& v, std::size_t expected, const char* name) {
    if (v.size() != expected)
        throw std::invalid_argument(std::string("decoder data: ") + name + " has " +
                                    std::to_string(v.size()) + " values, expected " +
                                    std::to_string(expected));
}

}  // namespace

std::shared_ptr<SfgHipLibrary> load_library(const std::filesystem::path& requested) {
    static std::mutex mutex;
    static std::shared_ptr<SfgHipLibrary> cached;
    std::lock_guard lock(mutex);
    const auto path = requested.empty() ? default_library_path() : requested;
    if (cached && cached->path == path.string()) return cached;
    cached = std::make_shared<SfgHipLibrary>(path);
    return cached;
}


DecoderExecutablePlan::DecoderExecutablePlan() = default;
DecoderExecutablePlan::~DecoderExecutablePlan() {
    if (device && device->ordinal >= 0) (void)hipSetDevice(device->ordinal);
}
DecoderExecutablePlan::DecoderExecutablePlan(DecoderExecutablePlan&&) noexcept = default;
DecoderExecutablePlan& DecoderExecutablePlan::operator=(DecoderExecutablePlan&&) noexcept = default;

// ---------------------------------------------------------------- public helpers

float round_to_bf16(float value) {
    const std::uint32_t bits = static_cast<std::uint32_t>(bf16_bits(value)) << 16;
    float out;
    std::memcpy(&out, &bits, sizeof out);
    return out;
}

double max_abs_error(const std::vector<float>& a, const std::vector<float>& b) {
    if (a.size() != b.size()) throw std::invalid_argument("max_abs_error: size mismatch");
    double worst = 0.0;
    for (std::size_t i = 0; i < a.size(); ++i)
        worst = std::max(worst, std::abs(static_cast<double>(a[i]) - static_cast<double>(b[i])));
    return worst;
}

std::string decoder_ffn_name(DecoderFFNKind kind) {
    return kind == DecoderFFNKind::Dense ? "dense_swiglu" : "moe";
}

std::string decoder_precision_name(DecoderPrecision precision) {
    switch (precision) {
        case DecoderPrecision::F32: return "f32";
        case DecoderPrecision::BF16: return "bf16";
        case DecoderPrecision::W8: return "w8";
    }
    return "?";
}

void validate(const DecoderConfig& c) {
    if (c.batch <= 0 || c.sequence <= 0 || c.hidden <= 0 || c.intermediate <= 0 ||
        c.query_heads <= 0 || c.kv_heads <= 0 || c.head_dim <= 0 ||
        c.hidden != c.query_heads * c.head_dim || c.query_heads % c.kv_heads != 0 ||
        !(c.rms_epsilon > 0.0F))
        throw std::invalid_argument("invalid decoder configuration");
    if (c.ffn == DecoderFFNKind::MoE && (c.experts <= 0 || c.top_k <= 0 || c.top_k > c.experts))
        throw std::invalid_argument("invalid decoder MoE configuration");
    if (c.context_sequence < 0) throw std::invalid_argument("invalid decoder context sequence");
    if (c.page_tokens <= 0) throw std::invalid_argument("invalid KV page size");
}

NamedDecoderConfig named_decoder_config(const std::string& name) {
    NamedDecoderConfig n;
    DecoderConfig& c = n.config;
    if (name == "c1") {
        c = {.batch = 1, .sequence = 128, .hidden = 256, .intermediate = 688, .query_heads = 4,
             .kv_heads = 2, .head_dim = 64, .rms_epsilon = 1.0e-6F};
        n.seed = 1000;
    } else if (name == "c2") {
        c = {.batch = 16, .sequence = 1, .hidden = 2048, .intermediate = 5632, .query_heads = 16,
             .kv_heads = 4, .head_dim = 128, .context_sequence = 4096,
             .precision = DecoderPrecision::BF16};
        n.seed = 2000;
    } else if (name == "c3") {
        c = {.batch = 4, .sequence = 512, .hidden = 2048, .intermediate = 1408, .query_heads = 16,
             .kv_heads = 4, .head_dim = 128, .ffn = DecoderFFNKind::MoE, .experts = 8, .top_k = 2,
             .precision = DecoderPrecision::BF16};
        n.seed = 3000;
        n.router_bias_std = 0.5F;
    } else if (name == "c4") {
        c = {.batch = 1, .sequence = 8192, .hidden = 4096, .intermediate = 14336,
             .query_heads = 32, .kv_heads = 8, .head_dim = 128, .precision = DecoderPrecision::BF16};
        n.seed = 4000;
    } else if (name == "c5") {
        c = {.batch = 64, .sequence = 1, .hidden = 4096, .intermediate = 14336,
             .query_heads = 32, .kv_heads = 8, .head_dim = 128, .ffn = DecoderFFNKind::MoE,
             .experts = 8, .top_k = 2, .context_sequence = 8192, .precision = DecoderPrecision::W8};
        n.seed = 5000;
    } else {
        throw std::invalid_argument("unknown decoder config " + name + " (expected c1..c5)");
    }
    return n;
}

DecoderData make_decoder_data(const DecoderConfig& c, std::uint64_t seed, float router_bias_std) {
    validate(c);
    constexpr float kWeightStd = 0.02F;
    const std::size_t H = c.hidden, I = c.intermediate, kvd = c.kv_width(), rows = c.rows();
    DecoderData d;
    d.input = normal(seed, 0, rows * H, 1.0F);
    d.rms1_weight.assign(H, 1.0F);
    d.rms2_weight.assign(H, 1.0F);
    d.query_weight = normal(seed, 2, H * H, kWeightStd);
    d.key_weight = normal(seed, 3, H * kvd, kWeightStd);
    d.value_weight = normal(seed, 4, H * kvd, kWeightStd);
    d.output_weight = normal(seed, 5, H * H, kWeightStd);
    if (c.ffn == DecoderFFNKind::MoE) {
        const std::size_t E = c.experts;
        d.moe.router_weight = normal(seed, 10, H * E, kWeightStd);
        if (router_bias_std > 0.0F) d.router_bias = normal(seed, 11, E, router_bias_std);
        d.moe.w1 = normal(seed, 12, E * H * I, kWeightStd);
        d.moe.w3 = normal(seed, 13, E * H * I, kWeightStd);
        d.moe.w2 = normal(seed, 14, E * I * H, kWeightStd);
    } else {
        d.gate_weight = normal(seed, 7, H * I, kWeightStd);
        d.up_weight = normal(seed, 8, H * I, kWeightStd);
        d.down_weight = normal(seed, 9, I * H, kWeightStd);
    }
    if (c.decode()) {
        const std::size_t kv = static_cast<std::size_t>(c.batch) * kvd * c.context_sequence;
        d.cached_key = normal(seed, 15, kv, 1.0F);
        d.cached_value = normal(seed, 16, kv, 1.0F);
        d.page_table = page_permutation(seed, static_cast<std::int64_t>(c.batch) * c.pages_per_sequence());
    }
    if (c.precision != DecoderPrecision::F32) {
        round_in_place(d.input);
        round_in_place(d.cached_key);
        round_in_place(d.cached_value);
    }
    if (c.precision == DecoderPrecision::BF16) {
        for (auto* v : {&d.query_weight, &d.key_weight, &d.value_weight, &d.output_weight,
                        &d.gate_weight, &d.up_weight, &d.down_weight, &d.moe.router_weight,
                        &d.moe.w1, &d.moe.w3, &d.moe.w2})
            round_in_place(*v);
    }
    return d;
}

// ---------------------------------------------------------------- dumps

std::string DecoderConstant::dump() const {
    std::ostringstream out;
    auto shape = [&](const std::vector<int>& s) {
        out << '[';
        for (std::size_t i = 0; i < s.size(); ++i) out << (i ? "x" : "") << s[i];
        out << ']';
    };
    out << name << " logical=";
    shape(logical_shape);
    out << " packed=";
    shape(packed_shape);
    out << " layout=" << layout << " bytes=" << bytes;
    return out.str();
}

std::string DecoderMemoryPlan::dump() const {
    std::ostringstream out;
    out << "memory naive_bytes=" << naive_bytes << " workspace_bytes=" << workspace_bytes
        << " constant_bytes=" << constant_bytes;
    return out.str();
}

std::string DecoderExecutablePlan::dump() const {
    const DecoderConfig& c = config;
    std::ostringstream out;
    out << "sfe.decoder_executable version=0.9.0 target=gfx950 ffn=" << decoder_ffn_name(c.ffn)
        << " hardware=\"" << hardware << "\" {\n"
        << "config batch=" << c.batch << " sequence=" << c.sequence << " hidden=" << c.hidden
        << " intermediate=" << c.intermediate << " query_heads=" << c.query_heads
        << " kv_heads=" << c.kv_heads << " head_dim=" << c.head_dim
        << " rms_epsilon=" << c.rms_epsilon << " rope_theta=" << c.rope_theta
        << " causal=" << c.causal << " experts=" << c.experts << " top_k=" << c.top_k
        << " context_sequence=" << c.context_sequence
        << " precision=" << decoder_precision_name(c.precision)
        << " page_tokens=" << c.page_tokens << '\n'
        << "library \"" << library_metadata << "\"\n"
        << policy.dump()
        << "\ncompile_ms=" << compile_milliseconds << "\nconstants {\n";
    for (const auto& constant : constants) out << "  " << constant.dump() << '\n';
    out << "}\n" << memory.dump() << "\nkernels {\n"
        << "  rmsnorm\n  qkv_gemm\n"
        << (c.decode() ? "  paged_decode_attention(split_kv)\n"
                       : "  split_rope\n  prefill_attention(io_aware)\n")
        << "  output_projection(+residual)\n  rmsnorm\n";
    if (c.ffn == DecoderFFNKind::Dense)
        out << "  gate_up(swiglu)\n  down(+residual)\n";
    else
        out << "  router(softmax,topk)\n  dispatch(histogram,prefix,scatter)\n"
               "  grouped_experts(w13 glu, w2)\n  combine(+residual)\n";
    out << "}\n}\n";
    return out.str();
}

std::string gemm_tile_name(int tile) {
    switch (tile) {
        case SFG_TILE_AUTO: return "auto";
        case SFG_TILE_256x256_PP: return "256x256pp";
        case SFG_TILE_256x256_W8: return "256x256w8";
        case SFG_TILE_256x256_W4: return "256x256w4";
        case SFG_TILE_256x128: return "256x128";
        case SFG_TILE_128x256: return "128x256";
        case SFG_TILE_128x128: return "128x128";
        case SFG_TILE_256x256_V: return "256x256v";
        default: return "tile" + std::to_string(tile);
    }
}

int parse_gemm_tile(const std::string& name) {
    for (int t = SFG_TILE_AUTO; t < SFG_TILE_COUNT; ++t)
        if (gemm_tile_name(t) == name) return t;
    throw std::invalid_argument("unknown GEMM tile " + name);
}

std::string DecoderPlanPolicy::dump() const {
    std::ostringstream out;
    out << "policy weight_layout="
        << (weight_layout < 0 ? "auto" : (weight_layout == SFG_LAYOUT_TILED ? "tiled16x8" : "nk"))
        << " kv_splits=" << (kv_splits > 0 ? std::to_string(kv_splits) : std::string("auto"))
        << " gemm_tile=" << gemm_tile_name(gemm_tile)
        << " attn_waves=" << (attn_waves > 0 ? std::to_string(attn_waves) : std::string("auto"));
    return out.str();
}

void DecoderExecutablePlan::apply_policy(const DecoderPlanPolicy& next) {
    if (!device) throw std::invalid_argument("decoder plan was not compiled");
    if (next.weight_layout >= 0 && next.weight_layout != policy.weight_layout)
        throw std::invalid_argument("apply_policy: the weight layout is fixed at compile time");
    if (next.kv_splits < 0 || next.gemm_tile < SFG_TILE_AUTO || next.gemm_tile >= SFG_TILE_COUNT ||
        (next.attn_waves != 0 && next.attn_waves != 4 && next.attn_waves != 8))
        throw std::invalid_argument("apply_policy: invalid policy " + next.dump());
    std::lock_guard lock(device->mutex);
    sfg_layer_desc& d = device->desc;
    const int old_splits = d.kv_splits;
    d.kv_splits = next.kv_splits;
    d.gemm_tile = next.gemm_tile;
    d.attn_waves = next.attn_waves;
    // The split-KV count sizes the decode partials: grow the workspace if needed.
    if (d.kv_splits != old_splits && device->lib->layer_workspace(&d) > device->workspace.bytes)
        memory.workspace_bytes = allocate_workspace(*device);
    policy.kv_splits = next.kv_splits;
    policy.gemm_tile = next.gemm_tile;
    policy.attn_waves = next.attn_waves;
}

void DecoderExecutablePlan::save(const std::filesystem::path& path) const {
    if (path.has_parent_path()) std::filesystem::create_directories(path.parent_path());
    std::ofstream output(path);
    if (!output) throw std::runtime_error("cannot write decoder executable plan: " + path.string());
    output << dump();
}

// ---------------------------------------------------------------- compile

namespace {

int weight_dtype(DecoderPrecision p) {
    switch (p) {
        case DecoderPrecision::F32: return SFG_F32;
        case DecoderPrecision::BF16: return SFG_BF16;
        case DecoderPrecision::W8: return SFG_I8;
    }
    return SFG_F32;
}

std::size_t weight_element_bytes(DecoderPrecision p) {
    return p == DecoderPrecision::F32 ? 4 : p == DecoderPrecision::BF16 ? 2 : 1;
}

struct Packer {
    DecoderExecutablePlan::Device& dev;
    DecoderPrecision precision;
    int layout;
    DeviceBuffer staging;
    std::vector<DecoderConstant>& constants;

    // One fp32 [k][n] block -> rows [row, row + n) of a packed [*][k] matrix.
    void block(const float* host, std::int64_t k, std::int64_t n, void* dst, float* scales,
               std::int64_t row) {
        const std::size_t bytes = static_cast<std::size_t>(k * n) * sizeof(float);
        if (staging.bytes < bytes) staging = DeviceBuffer(bytes);
        dev.upload(staging.ptr, host, bytes);
        char* out = static_cast<char*>(dst) + row * k * static_cast<std::int64_t>(weight_element_bytes(precision));
        if (precision == DecoderPrecision::W8)
            dev.lib->check(dev.lib->quantize_weight(staging.as<float>(), k, n,
                                                    reinterpret_cast<std::int8_t*>(out), scales + row,
                                                    layout, dev.stream),
                           "quantize weight");
        else
            dev.lib->check(dev.lib->pack_weight(staging.as<float>(), k, n, n, out,
                                                weight_dtype(precision), layout, dev.stream),
                           "pack weight");
        dev.sync();  // staging is reused by the next block
    }

    // Concatenates [k][n_i] blocks column-wise (concatenate_columns,
    // decoder_compiler.cpp:77-94) into one transposed [sum n_i][k] matrix.
    std::pair<void*, float*> matrix(const std::string& name, std::int64_t groups,
                                    const std::vector<std::pair<const float*, std::int64_t>>& parts,
                                    std::int64_t k, std::int64_t group_stride_elems,
                                    std::vector<int> logical) {
        std::int64_t rows = 0;
        for (const auto& p : parts) rows += p.second;
        const std::size_t bytes = static_cast<std::size_t>(groups * rows * k) * weight_element_bytes(precision);
        void* dst = dev.add(name, bytes);
        float* scales = nullptr;
        if (precision == DecoderPrecision::W8)
            scales = static_cast<float*>(dev.add(name + ".scales", static_cast<std::size_t>(groups * rows) * 4));
        for (std::int64_t g = 0; g < groups; ++g) {
            std::int64_t row = g * rows;
            for (const auto& [host, n] : parts) {
                block(host + g * group_stride_elems, k, n, dst, scales, row);
                row += n;
            }
        }
        DecoderConstant constant;
        constant.name = name;
        constant.logical_shape = std::move(logical);
        constant.packed_shape = groups > 1 ? std::vector<int>{static_cast<int>(groups), static_cast<int>(rows), static_cast<int>(k)}
                                           : std::vector<int>{static_cast<int>(rows), static_cast<int>(k)};
        constant.layout = std::string(layout == SFG_LAYOUT_TILED ? "tiled16x8" : "nk") + ":" +
                          decoder_precision_name(precision) + (scales ? "+scales" : "");
        constant.bytes = bytes + (scales ? static_cast<std::size_t>(groups * rows) * 4 : 0);
        constants.push_back(std::move(constant));
        return {dst, scales};
    }
};

// Paged pools from [B][Hkv][ctx][D] fp32: K [page][Hkv][pt][D] and V
// [page][Hkv][D][pt] (token-minor inside a page), bf16, page p of sequence b
// at physical slot table[b][p]; positions past the context stay zero.
// One paged pool in the layout the decode kernels read (K token-major, V
// token-minor inside a page), in the activation dtype: fp32 for the fp32
// path, bf16 bits otherwise.
template <typename T>
std::vector<T> build_pool(const DecoderConfig& c, const std::vector<float>& cache,
                          const std::vector<std::int32_t>& table, bool token_minor) {
    const std::int64_t pt = c.page_tokens, D = c.head_dim, Hkv = c.kv_heads, ctx = c.context_sequence;
    const std::int64_t pps = c.pages_per_sequence();
    const std::int64_t page_elems = Hkv * pt * D;
    std::vector<T> pool(static_cast<std::size_t>(table.size()) * page_elems, T{});
    parallel_for(c.batch * pps, [&](std::int64_t begin, std::int64_t end) {
        for (std::int64_t bp = begin; bp < end; ++bp) {
            const std::int64_t b = bp / pps, p = bp % pps;
            T* page = pool.data() + table[bp] * page_elems;
            for (std::int64_t h = 0; h < Hkv; ++h)
                for (std::int64_t t = 0; t < pt; ++t) {
                    const std::int64_t token = p * pt + t;
                    if (token >= ctx) break;
                    const float* src = cache.data() + ((b * Hkv + h) * ctx + token) * D;
                    for (std::int64_t e = 0; e < D; ++e) {
                        const std::int64_t at = token_minor ? (h * D + e) * pt + t : (h * pt + t) * D + e;
                        if constexpr (sizeof(T) == 4) page[at] = src[e];
                        else page[at] = bf16_bits(src[e]);
                    }
                }
        }
    });
    return pool;
}

}  // namespace

GpuTargetInfo query_target(const SfgHipLibrary& lib, int ordinal) {
    sfg_target_info t{};
    lib.check(lib.target_info(ordinal, &t), "target info");
    GpuTargetInfo g;
    g.architecture = t.architecture;
    g.wavefront = t.wavefront;
    g.compute_units = t.compute_units;
    g.xcds = t.xcds;
    g.simds_per_cu = t.simds_per_cu;
    g.lds_bytes_per_cu = static_cast<std::size_t>(t.lds_bytes_per_cu);
    g.l2_bytes_per_xcd = static_cast<std::size_t>(t.l2_bytes_per_xcd);
    g.hbm_bytes = static_cast<std::size_t>(t.hbm_bytes);
    g.engine_clock_ghz = t.engine_clock_ghz;
    g.hbm_gbps = t.hbm_gbps;
    g.mfma_bf16_tflops = t.mfma_bf16_tflops;
    g.valu_fp32_tflops = t.valu_fp32_tflops;
    return g;
}

std::string describe_hardware(const SfgHipLibrary& lib, int ordinal) {
    hipDeviceProp_t prop{};
    hip_check(hipGetDeviceProperties(&prop, ordinal), "hipGetDeviceProperties");
    return std::string(prop.name) + ' ' + query_target(lib, ordinal).str();
}

void fill_layer_desc(sfg_layer_desc& d, const DecoderConfig& c, const DecoderPlanPolicy& policy,
                     int pages_per_seq, int num_pages, bool use_routing_trace) {
    d = sfg_layer_desc{};
    d.abi = SFG_HIP_ABI_VERSION;
    d.batch = c.batch;
    d.sequence = c.sequence;
    d.hidden = c.hidden;
    d.intermediate = c.intermediate;
    d.query_heads = c.query_heads;
    d.kv_heads = c.kv_heads;
    d.head_dim = c.head_dim;
    d.rms_epsilon = c.rms_epsilon;
    d.rope_theta = c.rope_theta;
    d.causal = c.causal ? 1 : 0;
    d.ffn = c.ffn == DecoderFFNKind::MoE ? 1 : 0;
    d.experts = c.experts;
    d.top_k = c.top_k;
    d.context = c.context_sequence;
    d.page_tokens = c.page_tokens;
    d.pages_per_seq = pages_per_seq;
    d.num_pages = num_pages;
    d.act_dtype = c.precision == DecoderPrecision::F32 ? SFG_F32 : SFG_BF16;
    d.weight_dtype = weight_dtype(c.precision);
    d.kv_splits = policy.kv_splits;
    d.use_routing_trace = use_routing_trace ? 1 : 0;
    d.weight_layout = policy.weight_layout;
    d.gemm_tile = policy.gemm_tile;
    d.attn_waves = policy.attn_waves;
}

std::size_t allocate_workspace(DecoderExecutablePlan::Device& dev) {
    const std::size_t ws = dev.lib->layer_workspace(&dev.desc);
    if (ws == 0) dev.lib->check(SFG_ERR_INVALID_CONFIG, "decoder layer workspace");
    dev.workspace = DeviceBuffer(ws);
    hip_check(hipMemsetAsync(dev.workspace.ptr, 0, ws, dev.stream), "hipMemsetAsync");
    dev.sync();
    return ws;
}

DecoderExecutablePlan DecoderCompiler::compile(const DecoderConfig& config, const DecoderData& data,
                                               DecoderCompileOptions options) const {
    const auto started = std::chrono::steady_clock::now();
    validate(config);
    const DecoderConfig& c = config;
    const std::int64_t H = c.hidden, I = c.intermediate, D = c.head_dim, kvd = c.kv_width();
    const std::int64_t rows = c.rows(), E = c.experts;
    const bool moe = c.ffn == DecoderFFNKind::MoE;

    require_size(data.input, rows * H, "input");
    require_size(data.rms1_weight, H, "rms1_weight");
    require_size(data.rms2_weight, H, "rms2_weight");
    require_size(data.query_weight, H * H, "query_weight");
    require_size(data.key_weight, H * kvd, "key_weight");
    require_size(data.value_weight, H * kvd, "value_weight");
    require_size(data.output_weight, H * H, "output_weight");
    if (moe) {
        require_size(data.moe.router_weight, H * E, "moe.router_weight");
        require_size(data.moe.w1, E * H * I, "moe.w1");
        require_size(data.moe.w3, E * H * I, "moe.w3");
        require_size(data.moe.w2, E * I * H, "moe.w2");
        if (!data.router_bias.empty()) require_size(data.router_bias, E, "router_bias");
    } else {
        require_size(data.gate_weight, H * I, "gate_weight");
        require_size(data.up_weight, H * I, "up_weight");
        require_size(data.down_weight, I * H, "down_weight");
    }
    if (c.decode()) {
        const std::size_t kv = static_cast<std::size_t>(c.batch) * kvd * c.context_sequence;
        require_size(data.cached_key, kv, "cached_key");
        require_size(data.cached_value, kv, "cached_value");
    }

    DecoderExecutablePlan plan;
    plan.config = c;
    plan.policy = options.policy.value_or(DecoderPlanPolicy{});
    {
        const DecoderPlanPolicy& q = plan.policy;
        if (q.weight_layout < -1 || q.weight_layout > SFG_LAYOUT_TILED || q.kv_splits < 0 ||
            q.gemm_tile < SFG_TILE_AUTO || q.gemm_tile >= SFG_TILE_COUNT ||
            (q.attn_waves != 0 && q.attn_waves != 4 && q.attn_waves != 8))
            throw std::invalid_argument("invalid decoder plan policy: " + q.dump());
    }
    plan.device = std::make_unique<DecoderExecutablePlan::Device>();
    auto& dev = *plan.device;
    dev.lib = load_library(options.library);
    dev.ordinal = options.device;
    plan.library_metadata = dev.lib->metadata();
    hip_check(hipSetDevice(dev.ordinal), "hipSetDevice");
    hip_check(hipStreamCreate(&dev.stream), "hipStreamCreate");
    plan.hardware = describe_hardware(*dev.lib, dev.ordinal);

    // One weight layout for the whole plan: fragment-tiled when every product
    // runs on the decode GEMV kernels, [N][K] otherwise.
    int layout = SFG_LAYOUT_NK;
    if (c.precision != DecoderPrecision::F32) {
        // (and every product's width a multiple of 64, which each of the
        // GEMV kernels' 16-, 32- and 64-column tiles divides)
        const int64_t qkv_n = H + 2 * static_cast<int64_t>(c.kv_heads) * c.head_dim;
        bool tiled = dev.lib->preferred_layout(rows, H, 0) == SFG_LAYOUT_TILED &&
                     dev.lib->preferred_layout(rows, I, 0) == SFG_LAYOUT_TILED &&
                     qkv_n % 64 == 0 && H % 64 == 0 && I % 64 == 0;
        if (moe)
            tiled = tiled && dev.lib->preferred_layout(rows * c.top_k, H, 1) == SFG_LAYOUT_TILED &&
                    dev.lib->preferred_layout(rows * c.top_k, I, 1) == SFG_LAYOUT_TILED;
        layout = tiled ? SFG_LAYOUT_TILED : SFG_LAYOUT_NK;
        // A policy may ask for either layout where the decode GEMV kernels run
        // every product; the tiled layout feeds nothing else.
        if (plan.policy.weight_layout == SFG_LAYOUT_TILED && !tiled)
            throw std::invalid_argument("the tiled weight layout needs every product on the decode GEMV kernels");
        if (plan.policy.weight_layout >= 0) layout = plan.policy.weight_layout;
    } else if (plan.policy.weight_layout == SFG_LAYOUT_TILED) {
        throw std::invalid_argument("fp32 plans use the [N][K] weight layout");
    }
    plan.policy.weight_layout = layout;

    Packer pack{dev, c.precision, layout, DeviceBuffer(), plan.constants};
    sfg_layer_weights& w = dev.weights;
    auto vector_constant = [&](const std::string& name, const std::vector<float>& host) {
        void* p = dev.add(name, host.size() * sizeof(float));
        dev.upload(p, host.data(), host.size() * sizeof(float));
        plan.constants.push_back({name, {static_cast<int>(host.size())}, {static_cast<int>(host.size())},
                                  "f32", host.size() * sizeof(float)});
        return static_cast<const float*>(p);
    };
    w.rms1 = vector_constant("rms1_weight", data.rms1_weight);
    w.rms2 = vector_constant("rms2_weight", data.rms2_weight);
    {
        auto [p, s] = pack.matrix("packed_qkv_weight", 1,
                                  {{data.query_weight.data(), H}, {data.key_weight.data(), kvd},
                                   {data.value_weight.data(), kvd}},
                                  H, 0, {static_cast<int>(H), static_cast<int>(H + 2 * kvd)});
        w.w_qkv = p;
        w.s_qkv = s;
    }
    {
        auto [p, s] = pack.matrix("output_weight", 1, {{data.output_weight.data(), H}}, H, 0,
                                  {static_cast<int>(H), static_cast<int>(H)});
        w.w_o = p;
        w.s_o = s;
    }
    if (moe) {
        w.router = vector_constant("router_weight", data.moe.router_weight);
        if (!data.router_bias.empty()) w.router_bias = vector_constant("router_bias", data.router_bias);
        auto [p13, s13] = pack.matrix("expert_w13", E, {{data.moe.w1.data(), I}, {data.moe.w3.data(), I}}, H,
                                      H * I, {static_cast<int>(E), static_cast<int>(H), static_cast<int>(2 * I)});
        w.w13 = p13;
        w.s13 = s13;
        auto [p2, s2] = pack.matrix("expert_w2", E, {{data.moe.w2.data(), H}}, I, I * H,
                                    {static_cast<int>(E), static_cast<int>(I), static_cast<int>(H)});
        w.w2 = p2;
        w.s2 = s2;
    } else {
        auto [pg, sg] = pack.matrix("packed_gate_up_weight", 1,
                                    {{data.gate_weight.data(), I}, {data.up_weight.data(), I}}, H, 0,
                                    {static_cast<int>(H), static_cast<int>(2 * I)});
        w.w_gate_up = pg;
        w.s_gate_up = sg;
        auto [pd, sd] = pack.matrix("down_weight", 1, {{data.down_weight.data(), H}}, I, 0,
                                    {static_cast<int>(I), static_cast<int>(H)});
        w.w_down = pd;
        w.s_down = sd;
    }
    pack.staging = DeviceBuffer();

    // RoPE table [S][D/2][cos, sin], host-evaluated with the reference's
    // float expressions.
    std::vector<float> rope(static_cast<std::size_t>(c.sequence) * D);
    dev.lib->check(dev.lib->rope_table(rope.data(), c.sequence, D, c.rope_theta), "rope table");
    w.rope_table = vector_constant("rope_table", rope);

    int pages_per_seq = 0, num_pages = 0;
    if (c.decode()) {
        pages_per_seq = c.pages_per_sequence();
        num_pages = c.batch * pages_per_seq;
        std::vector<std::int32_t> table;
        if (data.page_table) {
            table = *data.page_table;
            if (table.size() != static_cast<std::size_t>(num_pages))
                throw std::invalid_argument("page table must hold batch x pages_per_sequence entries");
        } else {
            table.resize(num_pages);
            for (int i = 0; i < num_pages; ++i) table[i] = i;
        }
        std::vector<bool> used(num_pages, false);
        for (std::int32_t page : table) {
            if (page < 0 || page >= num_pages) throw std::invalid_argument("invalid physical KV page");
            if (used[page]) throw std::invalid_argument("physical KV page mapped twice");
            used[page] = true;
        }
        void* pt = dev.add("page_table", table.size() * 4);
        dev.upload(pt, table.data(), table.size() * 4);
        w.page_table = static_cast<const std::int32_t*>(pt);
        plan.constants.push_back({"page_table", {c.batch, pages_per_seq}, {c.batch, pages_per_seq}, "i32",
                                  table.size() * 4});
        const bool f32_pool = c.precision == DecoderPrecision::F32;
        for (const bool is_value : {false, true}) {
            const std::string name = is_value ? "v_pool" : "k_pool";
            const std::vector<float>& cache = is_value ? data.cached_value : data.cached_key;
            void* p = nullptr;
            std::size_t bytes = 0;
            auto place = [&](const auto& pool) {
                bytes = pool.size() * sizeof(pool[0]);
                p = dev.add(name, bytes);
                dev.upload(p, pool.data(), bytes);
                dev.sync();  // the host pool is released at scope end
            };
            if (f32_pool) place(build_pool<float>(c, cache, table, is_value));
            else place(build_pool<std::uint16_t>(c, cache, table, is_value));
            (is_value ? w.v_pool : w.k_pool) = p;
            plan.constants.push_back({name, {c.batch, c.kv_heads, c.context_sequence, static_cast<int>(D)},
                                      is_value ? std::vector<int>{num_pages, c.kv_heads, static_cast<int>(D), c.page_tokens}
                                               : std::vector<int>{num_pages, c.kv_heads, c.page_tokens, static_cast<int>(D)},
                                      f32_pool ? "paged:f32" : "paged:bf16", bytes});
        }
    }

    if (data.routing_trace) {
        const RoutingTrace& t = *data.routing_trace;
        if (!moe || t.expert_ids.size() != static_cast<std::size_t>(rows * c.top_k) ||
            t.expert_weights.size() != t.expert_ids.size())
            throw std::invalid_argument("routing trace does not match the layer");
        dev.trace_ids = DeviceBuffer(t.expert_ids.size() * 4);
        dev.trace_weights = DeviceBuffer(t.expert_weights.size() * 4);
        dev.upload(dev.trace_ids.ptr, t.expert_ids.data(), t.expert_ids.size() * 4);
        dev.upload(dev.trace_weights.ptr, t.expert_weights.data(), t.expert_weights.size() * 4);
    }

    fill_layer_desc(dev.desc, c, plan.policy, pages_per_seq, num_pages, data.routing_trace.has_value());
    const std::size_t ws = allocate_workspace(dev);

    plan.memory.workspace_bytes = ws;
    for (const auto& constant : plan.constants) plan.memory.constant_bytes += constant.bytes;
    // Every intermediate of execute_once materialised on its own.
    const std::int64_t act = c.precision == DecoderPrecision::F32 ? 4 : 2;
    const std::int64_t ffn_cols = moe ? static_cast<std::int64_t>(c.top_k) * 2 * I : 2 * I;
    plan.memory.naive_bytes = static_cast<std::size_t>(
        rows * H * (act + 4 + act + 4 + act + 4) + rows * (H + 2 * kvd) * 4 +
        (c.decode() ? 0 : 3 * rows * H * act) + rows * ffn_cols * 4 + rows * ffn_cols / 2 * act);
    plan.compile_milliseconds =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - started).count();
    return plan;
}

// ---------------------------------------------------------------- execute

DecoderBenchmarkResult execute_decoder_layer(const DecoderExecutablePlan& plan, const DecoderData& data,
                                             int warmup, int repetitions,
                                             const std::vector<float>* expected) {
    if (!plan.device) throw std::invalid_argument("decoder plan was not compiled");
    auto& dev = *plan.device;
    const DecoderConfig& c = plan.config;
    const std::size_t elems = static_cast<std::size_t>(c.rows()) * c.hidden;
    require_size(data.input, elems, "input");
    std::lock_guard lock(dev.mutex);
    hip_check(hipSetDevice(dev.ordinal), "hipSetDevice");

    DeviceBuffer x(elems * 4), out(elems * 4);
    dev.upload(x.ptr, data.input.data(), elems * 4);
    sfg_layer_io io{};
    io.x = x.as<float>();
    io.out = out.as<float>();
    if (dev.desc.use_routing_trace) {
        io.trace_ids = dev.trace_ids.as<std::int32_t>();
        io.trace_weights = dev.trace_weights.as<float>();
    }
    auto run = [&] {
        dev.lib->check(dev.lib->layer(&dev.desc, &dev.weights, &io, dev.workspace.ptr, dev.workspace.bytes,
                                      dev.stream),
                       "decoder layer");
    };
    for (int i = 0; i < std::max(0, warmup); ++i) run();
    dev.sync();

    void* events[SFG_NUM_MARKS] = {};
    dev.lib->check(dev.lib->events_create(SFG_NUM_MARKS, events), "events");
    io.stage_events = events;
    struct Stages {
        double total, attention, projection, norm_rope, ffn;
    };
    std::vector<Stages> measured;
    try {
        auto ms = [&](int a, int b) {
            float v = 0.0F;
            dev.lib->check(dev.lib->event_elapsed(events[a], events[b], &v), "event elapsed");
            return static_cast<double>(v);
        };
        for (int i = 0; i < std::max(1, repetitions); ++i) {
            run();
            dev.sync();
            Stages s{};
            s.total = ms(SFG_MARK_START, SFG_MARK_END);
            s.norm_rope = ms(SFG_MARK_START, SFG_MARK_NORM1) + ms(SFG_MARK_QKV, SFG_MARK_ROPE) +
                          ms(SFG_MARK_OPROJ, SFG_MARK_NORM2);
            s.projection = ms(SFG_MARK_NORM1, SFG_MARK_QKV) + ms(SFG_MARK_ATTN, SFG_MARK_OPROJ);
            s.attention = ms(SFG_MARK_ROPE, SFG_MARK_ATTN);
            s.ffn = ms(SFG_MARK_NORM2, SFG_MARK_END);
            measured.push_back(s);
        }
    } catch (...) {
        dev.lib->events_destroy(SFG_NUM_MARKS, events);
        throw;
    }
    dev.lib->events_destroy(SFG_NUM_MARKS, events);

    // Median by total time (decoder_compiler.cpp:684-687).
    std::sort(measured.begin(), measured.end(), [](const Stages& a, const Stages& b) { return a.total < b.total; });
    const Stages& med = measured[measured.size() / 2];
    DecoderBenchmarkResult r;
    r.milliseconds = med.total;
    r.attention_milliseconds = med.attention;
    r.projection_milliseconds = med.projection;
    r.norm_rope_milliseconds = med.norm_rope;
    r.ffn_milliseconds = med.ffn;
    // Residual adds are GEMM / combine epilogues on this target.
    r.residual_milliseconds = 0.0;
    r.dispatch_overhead_milliseconds =
        std::max(0.0, r.milliseconds - (r.attention_milliseconds + r.projection_milliseconds +
                                        r.norm_rope_milliseconds + r.ffn_milliseconds));
    r.tokens_per_second = r.milliseconds > 0.0 ? c.rows() * 1000.0 / r.milliseconds : 0.0;
    r.output.resize(elems);
    hip_check(hipMemcpyAsync(r.output.data(), out.ptr, elems * 4, hipMemcpyDeviceToHost, dev.stream),
              "hipMemcpyAsync");
    dev.sync();
    r.max_error = expected ? max_abs_error(r.output, *expected) : std::numeric_limits<double>::quiet_NaN();
    return r;
}


GpuTargetInfo GpuTargetInfo::detect(int device, const std::filesystem::path& library) {
    const auto lib = load_library(library);
    return query_target(*lib, device);
}

std::string GpuTargetInfo::str() const {
    std::ostringstream out;
    out << architecture << " wave" << wavefront << ' ' << compute_units << " CUs " << xcds << " XCDs "
        << (lds_bytes_per_cu >> 10) << " KiB LDS/CU " << (l2_bytes_per_xcd >> 20) << " MiB L2/XCD "
        << (hbm_bytes >> 30) << " GiB HBM " << std::fixed << std::setprecision(2) << engine_clock_ghz
        << " GHz";
    return out.str();
}

}  // namespace schedforge::hip
