// sfg-decoder-bench: the reference's realistic-profile benchmark driver
// (tools/schedforge-decoder-bench.cpp:14-114) for gfx950 plans.  Same options
// and report lines; profiles run at --precision (the reference's are fp32).
//
// Suites:
//   realistic   every profile of realistic_decoder_profiles()
//   optimizer   tiny-prefill-s128 and tiny-decode-kv512 with --optimize, as the
//               reference's suite; on this target the plan optimizer also runs
//               over the five benchmark configurations when --filter selects them
//   baseline    the five benchmark configurations c1..c5 (their own precisions)
// Extra options: --precision=f32|bf16|w8 (default bf16: this target's decode
// runs on a bf16 paged KV cache and its MoE layers on bf16 activations, so
// fp32 profiles of those kinds are recorded as skipped), --device=N,
// --compile-only (every profile analytical, no GPU touched).  The real-execution
// budgets default to a GPU's (5000 GFLOP, 16 GiB of weights) where the
// reference's default to a CPU's (1 GFLOP, 256 MiB).
#include "sfg_decoder.hpp"

#include <algorithm>
#include <cstdint>
#include <iomanip>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

namespace sh = schedforge::hip;

struct Options {
    std::string suite = "realistic";
    std::string output = "results/decoder_gpu.csv";
    int repetitions = 1;
    std::uint64_t max_real_flops = 5000ULL * 1000000000ULL;
    std::size_t max_real_weight_bytes = 16ULL * 1024 * 1024 * 1024;
    bool optimize = false;
    bool compile_only = false;
    std::string filter;
    sh::DecoderPrecision precision = sh::DecoderPrecision::BF16;
    int device = 0;
};

Options parse(int argc, char** argv) {
    Options o;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto value = [&](const char* key) { return a.substr(std::string(key).size()); };
        if (a.starts_with("--suite=")) o.suite = value("--suite=");
        else if (a.starts_with("--output=")) o.output = value("--output=");
        else if (a.starts_with("--threads=")) (void)std::stoi(value("--threads="));  // CPU knob, accepted
        else if (a.starts_with("--repetitions=")) o.repetitions = std::stoi(value("--repetitions="));
        else if (a.starts_with("--max-real-gflop="))
            o.max_real_flops = static_cast<std::uint64_t>(std::stod(value("--max-real-gflop=")) * 1.0e9);
        else if (a.starts_with("--max-weight-mib="))
            o.max_real_weight_bytes =
                static_cast<std::size_t>(std::stod(value("--max-weight-mib=")) * 1024.0 * 1024.0);
        else if (a.starts_with("--filter=")) o.filter = value("--filter=");
        else if (a.starts_with("--device=")) o.device = std::stoi(value("--device="));
        else if (a.starts_with("--precision=")) {
            const std::string p = value("--precision=");
            if (p == "f32") o.precision = sh::DecoderPrecision::F32;
            else if (p == "bf16") o.precision = sh::DecoderPrecision::BF16;
            else if (p == "w8") o.precision = sh::DecoderPrecision::W8;
            else throw std::invalid_argument("unknown precision " + p);
        } else if (a == "--optimize") o.optimize = true;
        else if (a == "--compile-only") o.compile_only = true;
        else if (a == "--help") {
            std::cout << "sfg-decoder-bench [--suite=realistic|optimizer|baseline]\n"
                         "  [--output=results/decoder_gpu.csv] [--repetitions=1]\n"
                         "  [--max-real-gflop=5000 --max-weight-mib=16384] [--filter=tiny-decode --optimize]\n"
                         "  [--precision=bf16|f32|w8 --device=0 --compile-only]\n";
            std::exit(0);
        } else {
            throw std::invalid_argument("unknown option: " + a);
        }
    }
    if (o.suite != "realistic" && o.suite != "optimizer" && o.suite != "baseline")
        throw std::invalid_argument("unknown suite: " + o.suite);
    if (o.suite == "optimizer") o.optimize = true;
    if (o.compile_only) {
        o.max_real_flops = 0;
        o.optimize = false;
    }
    return o;
}

}  // namespace

int main(int argc, char** argv) {
    Options options;
    try {
        options = parse(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 2;
    }
    try {
        auto profiles = options.suite == "baseline" ? sh::baseline_decoder_profiles()
                                                    : sh::realistic_decoder_profiles(options.precision);
        if (options.suite == "optimizer" && options.filter.empty())
            std::erase_if(profiles, [](const sh::DecoderBenchmarkProfile& p) {
                return p.name != "tiny-prefill-s128" && p.name != "tiny-decode-kv512";
            });
        if (!options.filter.empty())
            std::erase_if(profiles, [&](const sh::DecoderBenchmarkProfile& p) {
                return p.name.find(options.filter) == std::string::npos;
            });
        sh::DecoderCompileOptions compile;
        compile.device = options.device;
        std::vector<sh::DecoderBenchmarkRecord> records;
        records.reserve(profiles.size());
        for (const auto& profile : profiles) {
            std::cout << "[Profile] " << profile.name << " ... " << std::flush;
            auto record = sh::benchmark_decoder_profile(profile, options.max_real_flops,
                                                        options.max_real_weight_bytes, options.optimize,
                                                        options.repetitions, compile);
            std::cout << sh::decoder_evidence_name(record.evidence);
            if (record.evidence == sh::DecoderEvidenceKind::Measured)
                std::cout << ' ' << std::fixed << std::setprecision(3) << record.measured.milliseconds
                          << " ms, " << record.measured.tokens_per_second << " token/s, "
                          << record.selected_policy;
            else
                std::cout << " weight=" << profile.estimated_weight_bytes << " flops=" << profile.estimated_flops
                          << " estimate=" << std::fixed << std::setprecision(1)
                          << record.plan_cost.analytical_score << " us"
                          << (record.note.empty() ? "" : " (" + record.note + ")");
            if (record.hardware_measurements)
                std::cout << " optimizer=" << std::setprecision(3) << record.optimizer_speedup << "x/"
                          << record.hardware_measurements << " measurements";
            std::cout << '\n' << std::flush;
            records.push_back(std::move(record));
        }
        sh::write_decoder_benchmark_csv(options.output, records);
        if (options.optimize) {
            std::string candidates = options.output;
            const auto ext = candidates.rfind(".csv");
            if (ext != std::string::npos) candidates.insert(ext, "_candidates");
            else candidates += "_candidates.csv";
            sh::write_decoder_plan_candidates_csv(candidates, records);
            std::cout << "[Candidates] output=" << candidates << '\n';
        }
        const auto measured = std::count_if(records.begin(), records.end(), [](const auto& r) {
            return r.evidence == sh::DecoderEvidenceKind::Measured;
        });
        const auto skipped = std::count_if(records.begin(), records.end(), [](const auto& r) {
            return r.evidence == sh::DecoderEvidenceKind::Skipped;
        });
        std::cout << "[Summary] profiles=" << records.size() << " measured=" << measured
                  << " compile-only=" << records.size() - static_cast<std::size_t>(measured + skipped)
                  << " skipped=" << skipped << " output=" << options.output << '\n';
        return 0;
    } catch (const std::invalid_argument& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 2;
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 1;
    }
}
