// sfg-decoder: compile and run one decoder layer on an MI355X through the C++
// runtime, with the reference decoder driver's options and report sections
// (tools/schedforge-decoder.cpp:18-89).  The StableHLO input of the reference
// driver is not taken: the GPU target executes the fixed decoder-layer
// structure.  Synthetic inputs come from make_decoder_data's seeded generator.
//
// Extra options:
//   --config=c1..c5          one of the five benchmark configurations
//   --precision=f32|bf16|w8  --context=N  --page-tokens=N
//   --kv-splits=N --gemm-tile=NAME --attn-waves=N --weight-layout=auto|nk|tiled
//                            the plan policy (DecoderPlanPolicy)
//   --router-bias-std=S  --seed=N  --warmup=N  --device=N
//   --expect=FILE            raw fp32 [rows][hidden] to compare with (max_error)
//   --max-error=E            exit status 1 when max_error exceeds E (default 1e-3
//                            relative to max |expected|, as a fraction)
//   --dump-output=FILE       raw fp32 output
//   --dump-data=DIR          write the generated inputs as raw files and exit
//                            without touching the GPU
//   --package=DIR.sfe        also write the compiled plan as a .sfe GPU package
//   --load-package=DIR.sfe   run a packaged plan instead of compiling (shape
//                            options are taken from its manifest; --seed
//                            selects the input)
//   --inspect=DIR.sfe        validate a package without a GPU and print its
//                            manifest and plan (schedforge-aot inspect)
#include "sfg_decoder.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <optional>
#include <stdexcept>
#include <string>

namespace {

namespace sh = schedforge::hip;

struct Options {
    sh::DecoderConfig config;
    std::uint64_t seed = 71;
    float router_bias_std = 0.0F;
    sh::DecoderCompileOptions compile;
    int warmup = 1;
    int repetitions = 3;
    std::string output = "decoder_layer.sfe";
    std::string expect, dump_output, dump_data;
    std::string package, load_package, inspect;
    double max_relative_error = 1.0e-3;
};

int to_int(const std::string& s) { return std::stoi(s); }

sh::DecoderPlanPolicy& policy(Options& o) {
    if (!o.compile.policy) o.compile.policy.emplace();
    return *o.compile.policy;
}

Options parse(int argc, char** argv) {
    Options o;
    auto& c = o.config;
    auto value = [](const std::string& arg, const char* key) -> std::optional<std::string> {
        const std::string k(key);
        if (arg.rfind(k, 0) == 0) return arg.substr(k.size());
        return std::nullopt;
    };
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (auto v = value(a, "--config=")) {
            const auto named = sh::named_decoder_config(*v);
            c = named.config;
            o.seed = named.seed;
            o.router_bias_std = named.router_bias_std;
        } else if (auto v = value(a, "--batch=")) c.batch = to_int(*v);
        else if (auto v = value(a, "--sequence=")) c.sequence = to_int(*v);
        else if (auto v = value(a, "--hidden=")) c.hidden = to_int(*v);
        else if (auto v = value(a, "--intermediate=")) c.intermediate = to_int(*v);
        else if (auto v = value(a, "--q-heads=")) c.query_heads = to_int(*v);
        else if (auto v = value(a, "--kv-heads=")) c.kv_heads = to_int(*v);
        else if (auto v = value(a, "--head-dim=")) c.head_dim = to_int(*v);
        else if (auto v = value(a, "--experts=")) c.experts = to_int(*v);
        else if (auto v = value(a, "--top-k=")) c.top_k = to_int(*v);
        else if (auto v = value(a, "--context=")) c.context_sequence = to_int(*v);
        else if (auto v = value(a, "--page-tokens=")) c.page_tokens = to_int(*v);
        else if (auto v = value(a, "--rms-epsilon=")) c.rms_epsilon = std::stof(*v);
        else if (auto v = value(a, "--precision=")) {
            if (*v == "f32") c.precision = sh::DecoderPrecision::F32;
            else if (*v == "bf16") c.precision = sh::DecoderPrecision::BF16;
            else if (*v == "w8") c.precision = sh::DecoderPrecision::W8;
            else throw std::invalid_argument("unknown precision " + *v);
        } else if (auto v = value(a, "--router-bias-std=")) o.router_bias_std = std::stof(*v);
        else if (auto v = value(a, "--seed=")) o.seed = std::stoull(*v);
        else if (auto v = value(a, "--kv-splits=")) policy(o).kv_splits = to_int(*v);
        else if (auto v = value(a, "--gemm-tile=")) policy(o).gemm_tile = sh::parse_gemm_tile(*v);
        else if (auto v = value(a, "--attn-waves=")) policy(o).attn_waves = to_int(*v);
        else if (auto v = value(a, "--weight-layout=")) {
            if (*v == "auto") policy(o).weight_layout = -1;
            else if (*v == "nk") policy(o).weight_layout = SFG_LAYOUT_NK;
            else if (*v == "tiled") policy(o).weight_layout = SFG_LAYOUT_TILED;
            else throw std::invalid_argument("unknown weight layout " + *v);
        }
        else if (auto v = value(a, "--device=")) o.compile.device = to_int(*v);
        else if (auto v = value(a, "--warmup=")) o.warmup = to_int(*v);
        else if (auto v = value(a, "--repetitions=")) o.repetitions = to_int(*v);
        else if (auto v = value(a, "--expect=")) o.expect = *v;
        else if (auto v = value(a, "--max-error=")) o.max_relative_error = std::stod(*v);
        else if (auto v = value(a, "--dump-output=")) o.dump_output = *v;
        else if (auto v = value(a, "--dump-data=")) o.dump_data = *v;
        else if (auto v = value(a, "--package=")) o.package = *v;
        else if (auto v = value(a, "--load-package=")) o.load_package = *v;
        else if (auto v = value(a, "--inspect=")) o.inspect = *v;
        else if (a == "--moe") c.ffn = sh::DecoderFFNKind::MoE;
        else if (a == "--non-causal") c.causal = false;
        else if (a == "-o" && i + 1 < argc) o.output = argv[++i];
        else if (a == "--help") {
            std::cout << "sfg-decoder [--config=c1..c5] [--batch=1 --sequence=16 --hidden=64]\n"
                         "  [--intermediate=128 --q-heads=4 --kv-heads=2 --head-dim=16]\n"
                         "  [--moe --experts=4 --top-k=2 --router-bias-std=0] [--context=0 --page-tokens=16]\n"
                         "  [--precision=f32|bf16|w8 --kv-splits=0 --device=0 --seed=71]\n"
                         "  [--gemm-tile=auto|256x256pp|256x256w8|256x256w4|256x128|128x256|128x128]\n"
                         "  [--attn-waves=0|4|8 --weight-layout=auto|nk|tiled]\n"
                         "  [--warmup=1 --repetitions=3 --non-causal] [-o decoder.sfe]\n"
                         "  [--expect=FILE --max-error=1e-3 --dump-output=FILE --dump-data=DIR]\n"
                         "  [--package=DIR.sfe | --load-package=DIR.sfe | --inspect=DIR.sfe]\n";
            std::exit(0);
        } else {
            throw std::invalid_argument("unknown option: " + a);
        }
    }
    return o;
}

void write_raw(const std::string& path, const void* data, std::size_t bytes) {
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    f.write(static_cast<const char*>(data), static_cast<std::streamsize>(bytes));
}

template <typename T>
void write_vector(const std::string& dir, const std::string& name, const std::vector<T>& v) {
    if (!v.empty()) write_raw(dir + "/" + name + ".bin", v.data(), v.size() * sizeof(T));
}

std::vector<float> read_floats(const std::string& path, std::size_t count) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    std::vector<float> v(count);
    f.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(count * sizeof(float)));
    if (f.gcount() != static_cast<std::streamsize>(count * sizeof(float)))
        throw std::invalid_argument(path + " does not hold rows x hidden fp32 values");
    return v;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        Options o = parse(argc, argv);
        if (!o.inspect.empty()) {
            const auto m = sh::inspect_decoder_package(o.inspect);
            std::cout << "[Manifest]\n" << m.dump() << "\n[Plan]\n"
                      << std::ifstream(std::filesystem::path(o.inspect) / m.plan.path).rdbuf()
                      << "\n[Validation]\npackage valid: " << m.code_objects.size()
                      << " code objects, " << m.buffers.size() << " buffers, " << m.constants.bytes
                      << " constant bytes\n";
            return 0;
        }
        std::optional<sh::DecoderExecutablePlan> loaded;
        if (!o.load_package.empty()) {
            loaded.emplace(sh::load_decoder_package(o.load_package, o.compile.device));
            o.config = loaded->config;
        }
        sh::validate(o.config);
        const auto data = sh::make_decoder_data(o.config, o.seed, o.router_bias_std);
        if (!o.dump_data.empty()) {
            std::filesystem::create_directories(o.dump_data);
            const std::string& d = o.dump_data;
            write_vector(d, "input", data.input);
            write_vector(d, "query_weight", data.query_weight);
            write_vector(d, "key_weight", data.key_weight);
            write_vector(d, "value_weight", data.value_weight);
            write_vector(d, "output_weight", data.output_weight);
            write_vector(d, "gate_weight", data.gate_weight);
            write_vector(d, "up_weight", data.up_weight);
            write_vector(d, "down_weight", data.down_weight);
            write_vector(d, "router_weight", data.moe.router_weight);
            write_vector(d, "router_bias", data.router_bias);
            write_vector(d, "w1", data.moe.w1);
            write_vector(d, "w3", data.moe.w3);
            write_vector(d, "w2", data.moe.w2);
            write_vector(d, "cached_key", data.cached_key);
            write_vector(d, "cached_value", data.cached_value);
            if (data.page_table) write_vector(d, "page_table", *data.page_table);
            std::cout << "wrote generated inputs to " << d << '\n';
            return 0;
        }
        const auto plan = loaded ? std::move(*loaded) : sh::DecoderCompiler{}.compile(o.config, data, o.compile);
        plan.save(o.output);
        if (!o.package.empty()) {
            const auto m = sh::save_decoder_package(plan, o.package);
            std::cout << "[Package]\n" << o.package << ": " << m.code_objects.size() << " code objects, "
                      << m.buffers.size() << " buffers, " << m.constants.bytes << " constant bytes\n\n";
        }
        std::vector<float> expected;
        if (!o.expect.empty())
            expected = read_floats(o.expect, static_cast<std::size_t>(o.config.rows()) * o.config.hidden);
        const auto measured = sh::execute_decoder_layer(plan, data, o.warmup, o.repetitions,
                                                        o.expect.empty() ? nullptr : &expected);
        if (!o.dump_output.empty())
            write_raw(o.dump_output, measured.output.data(), measured.output.size() * sizeof(float));

        std::cout << "[Constants]\n";
        for (const auto& constant : plan.constants) std::cout << constant.dump() << '\n';
        std::cout << "\n[Memory]\n" << plan.memory.dump() << "\n\n[Plan Policy]\n"
                  << plan.policy.dump()
                  << "\n\n[Runtime]\nFFN: " << sh::decoder_ffn_name(o.config.ffn)
                  << "\nprecision: " << sh::decoder_precision_name(o.config.precision)
                  << std::fixed << std::setprecision(4)
                  << "\nexecution: " << measured.milliseconds << " ms\nattention: "
                  << measured.attention_milliseconds << " ms\nprojections: "
                  << measured.projection_milliseconds << " ms\nnorm+rope: "
                  << measured.norm_rope_milliseconds << " ms\nffn: " << measured.ffn_milliseconds
                  << " ms\ndispatch overhead: " << measured.dispatch_overhead_milliseconds
                  << " ms\n" << std::setprecision(1) << "tokens/s: " << measured.tokens_per_second
                  << std::setprecision(3) << "\ncompile: " << plan.compile_milliseconds << " ms\n";
        int status = 0;
        std::cout << "\n[Validation]\n";
        if (o.expect.empty()) {
            std::cout << "max error: n/a (no --expect)\n";
        } else {
            double scale = 0.0;
            for (float v : expected) scale = std::max(scale, static_cast<double>(std::fabs(v)));
            const double relative = measured.max_error / std::max(scale, 1.0e-30);
            std::cout << std::scientific << "max error: " << measured.max_error
                      << "\nmax relative error: " << relative << '\n';
            status = relative <= o.max_relative_error ? 0 : 1;
        }
        std::cout << "\n[Hardware]\n" << plan.hardware << '\n';
        return status;
    } catch (const std::invalid_argument& error) {
        std::cerr << "invalid argument: " << error.what() << '\n';
        return 2;
    } catch (const std::exception& error) {
        std::cerr << "error: " << error.what() << '\n';
        return 1;
    }
}
