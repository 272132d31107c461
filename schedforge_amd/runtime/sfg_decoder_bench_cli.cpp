// sfg-decoder-bench: runs the decoder-layer benchmark profiles on an MI355X and
// writes the benchmark CSV (and the plan-candidates CSV when the optimizer
// runs).  Its command line and report tags are the reference driver's
// interface (tools/schedforge-decoder-bench.cpp:14-114): the options --suite,
// --output, --repetitions, --threads, --max-real-gflop, --max-weight-mib,
// --filter, --optimize and the [Profile], [Candidates] and [Summary] lines.
//
// Suites (a table below):
//   realistic   realistic_decoder_profiles() at --precision
//   optimizer   the reference's optimizer pair (tiny-prefill-s128 and
//               tiny-decode-kv512) unless --filter picks others; forces --optimize
//   baseline    the five benchmark configurations c1..c5 at their own precisions
// Options of this target: --precision=f32|bf16|w8 (default bf16; f32 runs every
// profile on the fp32 path, decode over fp32 paged pools), --device=N, --compile-only (every
// profile analytical, no GPU touched), --expect-dir=DIR (a measured profile P
// with a file DIR/P.f32 of rows x hidden raw fp32 values gets max_error
// against it; the others report NaN).  Real-execution budgets default to a
// GPU's (5000 GFLOP, 16 GiB of weights).
#include "sfg_decoder.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <optional>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace {

namespace sh = schedforge::hip;
namespace fs = std::filesystem;

struct Settings {
    std::string suite = "realistic";
    fs::path output = "results/decoder_gpu.csv";
    int repetitions = 1;
    std::uint64_t flop_budget = 5000ULL * 1000000000ULL;
    std::size_t weight_budget = std::size_t(16) << 30;
    bool optimize = false;
    bool compile_only = false;
    std::string filter;
    sh::DecoderPrecision precision = sh::DecoderPrecision::BF16;
    int device = 0;
    fs::path expect_dir;
    bool help = false;
};

// One row per option.  Parsing and --help walk the same table; an option with
// a metavar takes "=VALUE", one without is a switch.
struct Flag {
    std::string_view name;
    std::string_view metavar;
    std::string_view help;
    void (*apply)(Settings&, const std::string&);
};

sh::DecoderPrecision precision_named(const std::string& v) {
    for (const auto p : {sh::DecoderPrecision::F32, sh::DecoderPrecision::BF16, sh::DecoderPrecision::W8})
        if (sh::decoder_precision_name(p) == v) return p;
    throw std::invalid_argument("unknown precision " + v);
}

const Flag kFlags[] = {
    {"--suite", "realistic|optimizer|baseline", "profile set",
     [](Settings& s, const std::string& v) { s.suite = v; }},
    {"--output", "FILE.csv", "benchmark CSV (default results/decoder_gpu.csv)",
     [](Settings& s, const std::string& v) { s.output = v; }},
    {"--repetitions", "N", "timed repetitions per profile (median kept)",
     [](Settings& s, const std::string& v) { s.repetitions = std::stoi(v); }},
    {"--threads", "N", "CPU thread count of the reference; accepted, unused on the GPU",
     [](Settings&, const std::string& v) { (void)std::stoi(v); }},
    {"--max-real-gflop", "G", "profiles above this many GFLOP are compile-only",
     [](Settings& s, const std::string& v) { s.flop_budget = static_cast<std::uint64_t>(std::stod(v) * 1e9); }},
    {"--max-weight-mib", "M", "profiles above this many MiB of weights are compile-only",
     [](Settings& s, const std::string& v) {
         s.weight_budget = static_cast<std::size_t>(std::stod(v) * double(std::size_t(1) << 20));
     }},
    {"--filter", "TEXT", "keep profiles whose name contains TEXT",
     [](Settings& s, const std::string& v) { s.filter = v; }},
    {"--optimize", "", "run the plan optimizer per profile",
     [](Settings& s, const std::string&) { s.optimize = true; }},
    {"--precision", "f32|bf16|w8", "arithmetic of the realistic profiles (default bf16)",
     [](Settings& s, const std::string& v) { s.precision = precision_named(v); }},
    {"--device", "N", "GPU ordinal",
     [](Settings& s, const std::string& v) { s.device = std::stoi(v); }},
    {"--compile-only", "", "analytical records only; no GPU is touched",
     [](Settings& s, const std::string&) { s.compile_only = true; }},
    {"--expect-dir", "DIR", "DIR/PROFILE.f32 expected outputs fill max_error",
     [](Settings& s, const std::string& v) { s.expect_dir = v; }},
    {"--help", "", "this text", [](Settings& s, const std::string&) { s.help = true; }},
};

struct Suite {
    std::string_view name;
    bool baseline_configs;                  // c1..c5 instead of the realistic list
    std::vector<std::string_view> default_names;  // kept when --filter is empty
    bool forces_optimize;
};

const std::vector<Suite>& suites() {
    static const std::vector<Suite> table = {
        {"realistic", false, {}, false},
        {"optimizer", false, {"tiny-prefill-s128", "tiny-decode-kv512"}, true},
        {"baseline", true, {}, false},
    };
    return table;
}

std::string usage() {
    std::ostringstream out;
    out << "sfg-decoder-bench";
    for (const Flag& f : kFlags)
        out << " [" << f.name << (f.metavar.empty() ? "" : "=") << f.metavar << ']';
    out << '\n';
    for (const Flag& f : kFlags) {
        std::string left(f.name);
        if (!f.metavar.empty()) left += "=" + std::string(f.metavar);
        out << "  " << left << std::string(left.size() < 38 ? 38 - left.size() : 1, ' ') << f.help << '\n';
    }
    return out.str();
}

Settings parse(int argc, char** argv) {
    Settings s;
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        const auto eq = arg.find('=');
        const std::string name = arg.substr(0, eq);
        const Flag* flag = nullptr;
        for (const Flag& f : kFlags)
            if (f.name == name) flag = &f;
        if (!flag) throw std::invalid_argument("unknown option: " + arg);
        const bool has_value = eq != std::string::npos;
        if (has_value == flag->metavar.empty())
            throw std::invalid_argument(std::string(flag->name) +
                                        (flag->metavar.empty() ? " takes no value" : " needs =VALUE"));
        flag->apply(s, has_value ? arg.substr(eq + 1) : std::string());
    }
    const auto suite = std::find_if(suites().begin(), suites().end(),
                                    [&](const Suite& t) { return t.name == s.suite; });
    if (suite == suites().end()) throw std::invalid_argument("unknown suite: " + s.suite);
    if (suite->forces_optimize) s.optimize = true;
    if (s.compile_only) {
        s.flop_budget = 0;
        s.optimize = false;
    }
    return s;
}

std::vector<sh::DecoderBenchmarkProfile> select_profiles(const Settings& s) {
    const Suite& suite = *std::find_if(suites().begin(), suites().end(),
                                       [&](const Suite& t) { return t.name == s.suite; });
    auto all = suite.baseline_configs ? sh::baseline_decoder_profiles()
                                      : sh::realistic_decoder_profiles(s.precision);
    const std::set<std::string_view> defaults(suite.default_names.begin(), suite.default_names.end());
    std::vector<sh::DecoderBenchmarkProfile> chosen;
    for (auto& p : all) {
        const bool keep = s.filter.empty() ? defaults.empty() || defaults.count(p.name) > 0
                                           : p.name.find(s.filter) != std::string::npos;
        if (keep) chosen.push_back(std::move(p));
    }
    return chosen;
}

// DIR/PROFILE.f32 as rows x hidden fp32 values, when the file exists.
std::optional<std::vector<float>> expected_output(const Settings& s, const sh::DecoderBenchmarkProfile& p) {
    if (s.expect_dir.empty()) return std::nullopt;
    const fs::path file = s.expect_dir / (p.name + ".f32");
    if (!fs::exists(file)) return std::nullopt;
    const std::size_t count = static_cast<std::size_t>(p.config.rows()) * p.config.hidden;
    if (fs::file_size(file) != count * sizeof(float))
        throw std::invalid_argument(file.string() + ": expected " + std::to_string(count) + " fp32 values");
    std::vector<float> values(count);
    std::ifstream in(file, std::ios::binary);
    in.read(reinterpret_cast<char*>(values.data()), static_cast<std::streamsize>(count * sizeof(float)));
    if (!in) throw std::runtime_error("cannot read " + file.string());
    return values;
}

std::string report(const sh::DecoderBenchmarkRecord& r) {
    std::ostringstream out;
    out << "[Profile] " << r.profile.name << ' ' << sh::decoder_evidence_name(r.evidence);
    out.setf(std::ios::fixed);
    if (r.evidence == sh::DecoderEvidenceKind::Measured) {
        out.precision(4);
        out << " latency_ms=" << r.measured.milliseconds;
        out.precision(1);
        out << " tokens_per_second=" << r.measured.tokens_per_second << " policy=" << r.selected_policy;
        if (!std::isnan(r.measured.max_error)) {
            out.precision(6);
            out << " max_error=" << r.measured.max_error;
        }
    } else {
        out.precision(1);
        out << " analytical_us=" << r.plan_cost.analytical_score << " flops=" << r.profile.estimated_flops
            << " weight_bytes=" << r.profile.estimated_weight_bytes;
        if (!r.note.empty()) out << " note=\"" << r.note << '"';
    }
    if (r.hardware_measurements > 0) {
        out.precision(3);
        out << " optimizer_speedup=" << r.optimizer_speedup << " measurements=" << r.hardware_measurements;
    }
    return out.str();
}

int run(const Settings& s) {
    const auto profiles = select_profiles(s);
    sh::DecoderCompileOptions compile;
    compile.device = s.device;
    std::vector<sh::DecoderBenchmarkRecord> records;
    for (const auto& profile : profiles) {
        const auto expected = expected_output(s, profile);
        records.push_back(sh::benchmark_decoder_profile(profile, s.flop_budget, s.weight_budget, s.optimize,
                                                        s.repetitions, compile,
                                                        expected ? &*expected : nullptr));
        std::cout << report(records.back()) << std::endl;
    }
    sh::write_decoder_benchmark_csv(s.output, records);
    if (s.optimize) {
        fs::path candidates = s.output;
        candidates.replace_filename(s.output.stem().string() + "_candidates" +
                                    (s.output.has_extension() ? s.output.extension().string() : ".csv"));
        sh::write_decoder_plan_candidates_csv(candidates, records);
        std::cout << "[Candidates] output=" << candidates.string() << '\n';
    }
    std::size_t by_kind[3] = {0, 0, 0};
    for (const auto& r : records) ++by_kind[static_cast<int>(r.evidence)];
    std::cout << "[Summary] profiles=" << records.size()
              << " measured=" << by_kind[static_cast<int>(sh::DecoderEvidenceKind::Measured)]
              << " compile-only=" << by_kind[static_cast<int>(sh::DecoderEvidenceKind::CompileOnly)]
              << " skipped=" << by_kind[static_cast<int>(sh::DecoderEvidenceKind::Skipped)]
              << " output=" << s.output.string() << '\n';
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    Settings settings;
    try {
        settings = parse(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 2;
    }
    if (settings.help) {
        std::cout << usage();
        return 0;
    }
    try {
        return run(settings);
    } catch (const std::invalid_argument& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 2;
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 1;
    }
}
