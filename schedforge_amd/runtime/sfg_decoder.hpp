// C++20 host runtime for the gfx950 decoder-layer backend.
//
// The reference's operator boundary for this path is the public C++ API of
// include/schedforge/decoder_compiler.h:
//   DecoderCompiler::compile(graph, config, data, options)   (205-214)
//   execute_decoder_layer(plan, data, warmup, repetitions)    (220-223)
// This header restates that API with the same type and field names for a plan
// whose target is an MI355X.  Everything below the plan is libsfg_hip.so's C ABI
// (include/sfg_hip.h), loaded with dlopen + dlsym and validated against its
// metadata string before the first call, as the reference's AOT loader does
// (src/aot_runtime.cpp:152-196, 259).
//
// Differences from the reference, all additive:
//   - DecoderConfig::precision selects fp32, bf16 or int8-weight plans (the
//     reference runs those as separate entry points).
//   - DecoderData carries an optional router bias and a paged-KV page table.
//   - The StableHLO graph argument of compile() is absent: the GPU target
//     executes the fixed decoder-layer structure the reference's fusion pass
//     checks for (decoder_compiler.cpp:531-533).
//   - execute_decoder_layer's max_error compares with a caller-supplied
//     expected output (the reference calls its scalar CPU layer there,
//     decoder_compiler.cpp:690); without one it is NaN.
// Errors follow the reference's convention: configuration, shape and guard
// violations throw std::invalid_argument; device and resource failures throw
// std::runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <limits>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <vector>

#include "sfg_hip.h"

namespace schedforge::hip {

enum class DecoderFFNKind { Dense, MoE };
// Arithmetic of a plan: all-fp32; bf16 weights and activations; int8
// per-output-channel weights with bf16 activations.
enum class DecoderPrecision { F32, BF16, W8 };

// decoder_compiler.h:17-32 (+ precision and page_tokens).
struct DecoderConfig {
    int batch = 1;
    int sequence = 16;
    int hidden = 64;
    int intermediate = 128;
    int query_heads = 4;
    int kv_heads = 2;
    int head_dim = 16;
    float rms_epsilon = 1.0e-5F;
    float rope_theta = 10000.0F;
    bool causal = true;
    DecoderFFNKind ffn = DecoderFFNKind::Dense;
    int experts = 4;
    int top_k = 2;
    int context_sequence = 0;
    DecoderPrecision precision = DecoderPrecision::F32;
    int page_tokens = 16;

    int rows() const { return batch * sequence; }
    int kv_width() const { return kv_heads * head_dim; }
    bool decode() const { return context_sequence > 0; }
    int pages_per_sequence() const { return (context_sequence + page_tokens - 1) / page_tokens; }
};

// Throws std::invalid_argument as validate() does (decoder_compiler.cpp:26-39).
void validate(const DecoderConfig& config);

// moe_compiler.h:51-59.
struct RoutingTrace {
    int tokens = 0;
    int experts = 0;
    int top_k = 0;
    std::vector<int> expert_ids;        // [tokens][top_k]
    std::vector<float> expert_weights;  // [tokens][top_k]
    std::vector<int> counts;            // [experts]
};

// moe_compiler.h:79-85.
struct MoeData {
    std::vector<float> input;
    std::vector<float> router_weight;  // [H][E]
    std::vector<float> w1;             // [E][H][I]
    std::vector<float> w3;             // [E][H][I]
    std::vector<float> w2;             // [E][I][H]
};

// decoder_compiler.h:34-49: host fp32 tensors in the reference's layouts
// ([K][N] weights, [B][Hkv][ctx][D] cached K/V).
struct DecoderData {
    std::vector<float> input;  // [B*S][H]
    std::vector<float> rms1_weight;
    std::vector<float> query_weight;
    std::vector<float> key_weight;
    std::vector<float> value_weight;
    std::vector<float> output_weight;
    std::vector<float> rms2_weight;
    std::vector<float> gate_weight;
    std::vector<float> up_weight;
    std::vector<float> down_weight;
    MoeData moe;
    std::vector<float> cached_key;
    std::vector<float> cached_value;
    std::optional<RoutingTrace> routing_trace;
    std::vector<float> router_bias;              // [E], empty: none
    std::optional<std::vector<int32_t>> page_table;  // [B][pages_per_seq]; default identity
};

// decoder_compiler.h:55-65.  The reference's policy picks CPU schedule knobs
// (attention intermediate layout, schedule family, core placement, threads);
// an MI355X plan chooses between kernel variants instead.  Every policy
// computes the same layer: GEMM tiles and flash-prefill block heights give
// bit-identical outputs, the weight layout only reorders bytes, and the
// split-KV count changes the softmax merge order (fp32 rounding only).
struct DecoderPlanPolicy {
    int weight_layout = -1;         // SFG_LAYOUT_NK / SFG_LAYOUT_TILED; -1: per shape
    int kv_splits = 0;              // decode split-KV count; 0: per shape
    int gemm_tile = SFG_TILE_AUTO;  // sfg_gemm_tile of the bf16 prefill / expert GEMMs
    int attn_waves = 0;             // bf16 flash prefill: 4 or 8 waves; 0: by grid size
    std::string dump() const;
    bool operator==(const DecoderPlanPolicy&) const = default;
};
std::string gemm_tile_name(int tile);
// Inverse of gemm_tile_name; throws std::invalid_argument for an unknown name.
int parse_gemm_tile(const std::string& name);

// decoder_compiler.h:133-139, reduced to what a GPU plan uses.
struct DecoderCompileOptions {
    int device = 0;
    std::optional<DecoderPlanPolicy> policy;  // empty: every field per shape
    std::filesystem::path library; // libsfg_hip.so; empty: beside this library
};

// decoder_compiler.h:67-74.
struct DecoderConstant {
    std::string name;
    std::vector<int> logical_shape;
    std::vector<int> packed_shape;
    std::string layout;
    std::size_t bytes = 0;
    std::string dump() const;
};

// decoder_compiler.h:76-80.
struct DecoderMemoryPlan {
    std::size_t naive_bytes = 0;      // every intermediate materialised separately
    std::size_t workspace_bytes = 0;  // the layer's planned workspace
    std::size_t constant_bytes = 0;   // packed weights, KV pools, tables
    std::string dump() const;
};

// decoder_compiler.h:119-130.
struct DecoderBenchmarkResult {
    double milliseconds = 0.0;
    double attention_milliseconds = 0.0;
    double projection_milliseconds = 0.0;
    double norm_rope_milliseconds = 0.0;
    double ffn_milliseconds = 0.0;
    double residual_milliseconds = 0.0;
    double dispatch_overhead_milliseconds = 0.0;
    double tokens_per_second = 0.0;
    double max_error = std::numeric_limits<double>::quiet_NaN();  // NaN: nothing to compare with
    std::vector<float> output;
};

// The GPU target of a plan: the counterpart of the reference's TargetInfo
// (include/schedforge/schedforge.h:15-34), which TargetInfo::detect() fills
// for the host CPU (src/target.cpp:8-17).  detect() queries the device through
// sfg_hip_target_info_v1: architecture, CUs, XCDs, LDS, L2, clock, HBM, and
// the peaks those imply.
struct GpuTargetInfo {
    std::string architecture;
    int wavefront = 64;
    int compute_units = 0;
    int xcds = 0;
    int simds_per_cu = 4;
    std::size_t lds_bytes_per_cu = 0;
    std::size_t l2_bytes_per_xcd = 0;
    std::size_t hbm_bytes = 0;
    double engine_clock_ghz = 0.0;
    double hbm_gbps = 0.0;
    double mfma_bf16_tflops = 0.0;
    double valu_fp32_tflops = 0.0;
    // `library`: libsfg_hip.so to query (empty: beside this library).
    static GpuTargetInfo detect(int device = 0, const std::filesystem::path& library = {});
    std::string str() const;
};

class SfgHipLibrary;
struct DeviceBuffer;

// decoder_compiler.h:97-117: an immutable, device-resident plan.  Owns the
// packed weights, the paged KV pools, the RoPE table and the workspace.
class DecoderExecutablePlan {
public:
    DecoderConfig config;
    std::vector<DecoderConstant> constants;
    DecoderMemoryPlan memory;
    std::string hardware;
    std::string library_metadata;
    DecoderPlanPolicy policy;  // weight_layout resolved to the packed layout
    double compile_milliseconds = 0.0;

    DecoderExecutablePlan();
    ~DecoderExecutablePlan();
    DecoderExecutablePlan(DecoderExecutablePlan&&) noexcept;
    DecoderExecutablePlan& operator=(DecoderExecutablePlan&&) noexcept;
    DecoderExecutablePlan(const DecoderExecutablePlan&) = delete;
    DecoderExecutablePlan& operator=(const DecoderExecutablePlan&) = delete;

    std::string dump() const;
    void save(const std::filesystem::path& path) const;
    // Switches the kernel variants of a compiled plan without recompiling:
    // kv_splits, gemm_tile and attn_waves change, the packed weights stay.  A
    // policy naming another weight layout than the packed one throws
    // std::invalid_argument (that needs DecoderCompiler::compile); -1 keeps it.
    void apply_policy(const DecoderPlanPolicy& policy);

    struct Device;
    std::unique_ptr<Device> device;  // buffers, descriptor, stream
};

class DecoderCompiler {
public:
    DecoderExecutablePlan compile(const DecoderConfig& config, const DecoderData& data,
                                  DecoderCompileOptions options = {}) const;
};

// The reference's decoder_compiler.cpp:675-692: warmup, timed repetitions,
// median by time, tokens/s = rows * 1000 / ms, per-stage times from device
// events.  `expected` (optional) fills max_error as max |output - expected|
// (runtime.cpp:628-635).
DecoderBenchmarkResult execute_decoder_layer(const DecoderExecutablePlan& plan,
                                             const DecoderData& data, int warmup = 1,
                                             int repetitions = 5,
                                             const std::vector<float>* expected = nullptr);

// ---------------------------------------------------------------- .sfe packages
//
// A compiled plan as an inspectable directory with a .sfe suffix, after the
// reference's AOT package format 1 (src/aot_runtime.cpp:217-316,
// docs/AOT_DEPLOYMENT.md:6-35), carrying what a GPU plan needs:
//   manifest.sfe      key=value: format, ABI, target, configuration, policy,
//                     buffer table, file and code-object checksums
//   plan.sfe          DecoderExecutablePlan::dump()
//   libsfg_hip.so     the host + device library the plan was compiled against
//   kernels/NN.gfx950.hsaco  the gfx950 code objects embedded in that library
//                     (the ones the HIP runtime loads), one per translation unit
//   constants.bin     device bytes of every plan buffer (packed weights, int8
//                     scales, RoPE table, page table, paged K/V pools, routing
//                     trace) at 256-byte aligned offsets
// Checksums are FNV-1a 64-bit as 16 hex digits (aot_runtime.cpp:26-35).
// Loading validates the format version, ABI, target, every checksum, the
// library's embedded metadata (sfg_hip_metadata_v1 and its ABI version) and
// that the library's embedded code objects are the packaged ones, then the
// device architecture; any mismatch throws std::runtime_error, with no
// fallback to recompilation.  Nothing is recompiled on load.
struct DecoderPackageFile {
    std::string path;  // relative to the package directory
    std::size_t bytes = 0;
    std::string checksum;
};
struct DecoderPackageCodeObject {
    DecoderPackageFile file;
    std::string target_id;  // offload bundle id, e.g. hipv4-amdgcn-amd-amdhsa--gfx950
};
struct DecoderPackageBuffer {
    std::string name;
    std::size_t offset = 0;
    std::size_t bytes = 0;
    std::string checksum;
};
struct DecoderPackageManifest {
    int format_version = 1;
    std::string schedforge_version;
    std::string abi;     // sfg_hip_decoder_layer_v1
    std::string symbol;  // the entry point resolved in the packaged library
    std::string target;  // gfx950
    int library_abi = 0;
    std::string library_metadata;
    DecoderConfig config;
    DecoderPlanPolicy policy;
    int pages_per_seq = 0;
    int num_pages = 0;
    bool routing_trace = false;
    std::size_t workspace_bytes = 0;
    std::size_t naive_bytes = 0;
    DecoderPackageFile plan, library, constants;
    std::vector<DecoderPackageCodeObject> code_objects;
    std::vector<DecoderPackageBuffer> buffers;
    std::vector<DecoderConstant> constant_table;

    std::string dump() const;
    // Throws std::runtime_error on an unknown format, ABI or a missing,
    // duplicate or malformed field (aot_runtime.cpp:97-121, 167-199).
    static DecoderPackageManifest parse(const std::string& text);
};

// FNV-1a 64-bit of a byte range as 16 lower-case hex digits.
std::string package_checksum(const void* data, std::size_t bytes);

// The gfx950 code objects inside a library's .hip_fatbin section, in link order
// (ELF section table, then the clang offload bundles it holds).
struct EmbeddedCodeObject {
    std::string target_id;
    std::vector<unsigned char> bytes;
};
std::vector<EmbeddedCodeObject> embedded_code_objects(const std::filesystem::path& library);

// Writes `plan` to `path` (which must end in .sfe) through a temporary
// directory renamed into place; returns the manifest written.
DecoderPackageManifest save_decoder_package(const DecoderExecutablePlan& plan,
                                            const std::filesystem::path& path);
// Validates a package without touching a GPU: manifest, file checksums, the
// packaged library's embedded metadata and code objects.
DecoderPackageManifest inspect_decoder_package(const std::filesystem::path& path);
// inspect_decoder_package, then the device's architecture, then the buffers
// uploaded to `device` and the plan rebuilt around the packaged library.
DecoderExecutablePlan load_decoder_package(const std::filesystem::path& path, int device = 0);

// Seeded synthetic inputs: a counter-based generator (SplitMix64 keyed by
// seed and tensor id, Box-Muller in double) with activations N(0,1), weights
// N(0,0.02), norm gains 1, cached K/V N(0,1), router bias N(0,router_bias_std)
// when positive, and a seeded Fisher-Yates page permutation.  bf16 plans round
// inputs, weights and the KV cache to bf16; int8 plans round inputs and the
// KV cache.  Tensor ids: x 0, rms1 1, Wq 2, Wk 3, Wv 4, Wo 5, rms2 6, Wg 7,
// Wu 8, Wd 9, router 10, router bias 11, W1 12, W3 13, W2 14, K 15, V 16,
// page permutation 17.
DecoderData make_decoder_data(const DecoderConfig& config, std::uint64_t seed,
                              float router_bias_std = 0.0F);

// The five benchmark configurations by name ("c1" ... "c5"), with their
// seeds (1000 c) and router bias std.
struct NamedDecoderConfig {
    DecoderConfig config;
    std::uint64_t seed = 0;
    float router_bias_std = 0.0F;
};
NamedDecoderConfig named_decoder_config(const std::string& name);

std::string decoder_ffn_name(DecoderFFNKind kind);
std::string decoder_precision_name(DecoderPrecision precision);
double max_abs_error(const std::vector<float>& a, const std::vector<float>& b);
float round_to_bf16(float value);

// ---------------------------------------------------------------- plan optimizer
//
// ExecutablePlanOptimizer (decoder_compiler.h:140-176, decoder_compiler.cpp:
// 726-861) over MI355X plan policies.  The search is the reference's:
// compile and measure the default plan (the baseline), score every candidate
// policy with an analytical model, measure the `measurement_budget` best
// scored, and when one beats the baseline confirm with three interleaved
// baseline / winner measurements (medians kept); the baseline stays unless its
// confirmed median is slower.  The analytical score is a roofline estimate of
// the layer in microseconds on this GPU (see GpuCostModel) in place of the
// reference's CPU penalties.  Candidates that share the packed weight layout
// reuse one compiled plan (apply_policy): only a layout change recompiles.

// decoder_compiler.h:140-147 (+ estimated_microseconds, the model's layer time).
struct DecoderPlanCost {
    double measured_milliseconds = 0.0;
    double analytical_score = 0.0;
    std::size_t workspace_bytes = 0;
    std::size_t materialization_bytes = 0;
    bool measured = false;
    std::string dump() const;
};

struct DecoderPlanCandidate {
    DecoderPlanPolicy policy;
    DecoderPlanCost cost;
};

// decoder_compiler.h:154-162.
struct DecoderOptimizationResult {
    DecoderExecutablePlan plan;
    DecoderPlanCost baseline;
    DecoderPlanCost winner;
    std::vector<DecoderPlanCandidate> candidates;  // [0] is the baseline
    std::size_t hardware_measurements = 0;
    double speedup = 1.0;
    std::string dump() const;
};

// Machine constants of the analytical model: MI355X spec peaks, derated by
// what this build's kernels reach on the box (calibration runs of the
// benchmark; the values are the model's only inputs besides the shape).
struct GpuCostModel {
    // Spec figures of the target; for_target() takes them from a detected
    // GpuTargetInfo (CUs, published HBM bandwidth, MFMA and VALU peaks).
    static GpuCostModel for_target(const GpuTargetInfo& target);
    int compute_units = 256;
    double hbm_bytes_per_second = 8.0e12;
    double mfma_bf16_flops = 2.5e15;
    double valu_fp32_flops = 157.3e12;
    double launch_microseconds = 2.5;  // per kernel on a busy stream
    // fraction of peak a kernel family sustains inside a full wave of tiles
    double hbm_efficiency = 0.68;
    double gemv_tiled_efficiency = 0.48;
    double gemv_nk_efficiency = 0.40;
    double fp32_gemm_efficiency = 0.30;
    double flash_efficiency = 0.42;
    // per sfg_gemm_tile: efficiency of one full wave of tiles
    double tile_efficiency[SFG_TILE_COUNT] = {0.0, 0.43, 0.45, 0.42, 0.44, 0.40, 0.36, 0.49};
};

class ExecutablePlanOptimizer {
public:
    explicit ExecutablePlanOptimizer(GpuCostModel model = {});
    // The candidate policies for a configuration (the reference enumerates its
    // policy space the same way, decoder_compiler.cpp:754-781): weight layouts
    // and split-KV counts for decode steps, GEMM tiles and flash-prefill block
    // heights for bf16 prefill.  The first is the default policy.
    std::vector<DecoderPlanPolicy> policies(const DecoderConfig& config) const;
    // Analytical cost of a policy; needs no GPU (compile-only records use it).
    DecoderPlanCost evaluate(const DecoderConfig& config, const DecoderPlanPolicy& policy) const;
    DecoderPlanCost evaluate(const DecoderExecutablePlan& plan) const;
    DecoderOptimizationResult optimize(const DecoderConfig& config, const DecoderData& data,
                                       int measurement_budget = 8, int repetitions = 2,
                                       const DecoderCompileOptions& options = {}) const;
    const GpuCostModel& model() const { return model_; }

private:
    GpuCostModel model_;
};

// ---------------------------------------------------------------- profile harness
//
// The reference's realistic-profile harness (decoder_compiler.h:178-238,
// decoder_compiler.cpp:863-1060) on the GPU: the same profile list, evidence
// classes and CSV schemas, with GPU columns appended after the reference's.

// moe_compiler.h (RoutingDistribution): expert draw weights 1 (uniform) or
// 1 / (e + 1)^0.8 (moderate) or ^1.6 (heavy), top-k distinct experts per token
// drawn by weight, each weighted 1 / k (moe_compiler.cpp:457-488).
enum class RoutingDistribution { Uniform, ModerateSkew, HeavySkew };
std::string routing_distribution_name(RoutingDistribution distribution);
RoutingTrace make_routing_trace(int tokens, int experts, int top_k,
                                RoutingDistribution distribution, std::uint64_t seed);

enum class DecoderEvidenceKind { Measured, CompileOnly, Skipped };
std::string decoder_evidence_name(DecoderEvidenceKind kind);

// decoder_compiler.h:180-187.
struct DecoderBenchmarkProfile {
    std::string name;
    DecoderConfig config;
    RoutingDistribution routing = RoutingDistribution::Uniform;
    std::uint64_t estimated_flops = 0;
    std::size_t estimated_weight_bytes = 0;
    std::size_t estimated_activation_bytes = 0;
};

// decoder_compiler.h:189-204 (+ the optimizer's policy spread).
struct DecoderBenchmarkRecord {
    DecoderBenchmarkProfile profile;
    DecoderEvidenceKind evidence = DecoderEvidenceKind::Skipped;
    DecoderBenchmarkResult measured;
    DecoderPlanCost plan_cost;
    double compile_milliseconds = 0.0;
    double llvm_compile_milliseconds = 0.0;  // always 0: nothing is JIT-compiled
    double memory_planning_milliseconds = 0.0;
    double optimizer_speedup = 1.0;
    double optimizer_baseline_milliseconds = 0.0;
    std::size_t hardware_measurements = 0;
    std::string selected_policy;
    std::vector<DecoderPlanCandidate> optimizer_candidates;
    std::string note;
};

// decoder_compiler.cpp:863-903: FLOPs (non-causal attention, as the reference
// counts), weight bytes at the profile's precision, activation bytes.
DecoderBenchmarkProfile make_decoder_profile(std::string name, DecoderConfig config,
                                             RoutingDistribution routing = RoutingDistribution::Uniform);
// decoder_compiler.cpp:905-930: tiny / medium / large dense prefill (S 128,
// 512, 2048) and decode (KV 128, 512, 2048, 4096), and the tiny MoE layer
// under three routing distributions, at the given precision.
std::vector<DecoderBenchmarkProfile> realistic_decoder_profiles(
    DecoderPrecision precision = DecoderPrecision::F32);
// The five benchmark configurations c1..c5 as profiles.
std::vector<DecoderBenchmarkProfile> baseline_decoder_profiles();
// decoder_compiler.cpp:932-987: compile-only (analytical cost, no GPU) above
// the FLOP or weight budget, else compile, optionally optimise, and measure.
// Configurations the GPU target does not lower are recorded as Skipped with
// the reason.
// `expected` (optional, rows x hidden) fills the record's max_error; without
// it max_error is NaN.
DecoderBenchmarkRecord benchmark_decoder_profile(const DecoderBenchmarkProfile& profile,
                                                 std::uint64_t max_real_flops,
                                                 std::size_t max_real_weight_bytes,
                                                 bool optimize_plan, int repetitions = 2,
                                                 const DecoderCompileOptions& options = {},
                                                 const std::vector<float>* expected = nullptr);
// decoder_compiler.cpp:989-1030 and 1032-1058: the reference's column lists,
// then precision, layer_tflops and layer_gbps (benchmark) and the GPU policy
// fields in place of the CPU ones (candidates).
void write_decoder_benchmark_csv(const std::filesystem::path& path,
                                 const std::vector<DecoderBenchmarkRecord>& records);
void write_decoder_plan_candidates_csv(const std::filesystem::path& path,
                                       const std::vector<DecoderBenchmarkRecord>& records);

}  // namespace schedforge::hip
