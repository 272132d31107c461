// Test infrastructure only: a C entry point over the reference's own CPU GEMM
// runtime, compiled from the reference sources where they lie (see the `ref`
// target of oracle/Makefile).  It lets the tests check the oracle's
// sfgo_matmul against the reference's execute() bit for bit, and lets the
// bench time the reference's GEMMs beside the oracle's.  Nothing in the
// product links or loads it.
//
// The schedule is the one the reference decoder gives every projection GEMM:
// decoder_schedule() (reference src/decoder_compiler.cpp:196-208), restated
// here because decoder_compiler.cpp itself cannot be built without LLVM.  The
// GEMM is planned with apply_schedule() and run with execute() exactly as
// the decoder's run step does (src/decoder_compiler.cpp:230, 554-559).
#include "schedforge/schedforge.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

namespace {

// decoder_schedule(): family 0 = Latency, 1 = Throughput.
schedforge::Schedule decoder_gemm_schedule(int family, int threads, int vector_width) {
    schedforge::Schedule s;
    const bool latency = family == 0;
    s.threads = std::max(1, threads);
    s.pin_threads = false;  // placement changes timing, not results
    s.bm = latency ? 8 : 32;
    s.bn = latency ? 32 : 128;
    s.bk = latency ? 32 : 64;
    s.mr = 4;
    s.nr = std::max(1, vector_width);
    s.vector_width = std::max(1, vector_width);
    s.fused = true;
    return s;
}

}  // namespace

extern "C" {

// c[m][n] = a[m][k] @ b[k][n], all row-major fp32 (no bias, no ReLU: the
// decoder's projections).  The reference's Problem holds int extents.
// Returns 0, or 1 on a bad extent or if the reference runtime threw (its
// message is dropped: this is a checker).
int sfgr_decoder_gemm(const float* a, const float* b, float* c, int m, int n, int k, int family,
                      int threads) {
    if (m <= 0 || n <= 0 || k <= 0) return 1;
    try {
        const schedforge::Problem problem{m, n, k, false, false};
        const auto loop = schedforge::apply_schedule(
            problem, decoder_gemm_schedule(family, threads, schedforge::TargetInfo::detect().vector_width));
        schedforge::TensorData data;
        data.a.assign(a, a + static_cast<int64_t>(m) * k);
        data.b.assign(b, b + static_cast<int64_t>(k) * n);
        std::vector<float> out;
        schedforge::execute(loop, data, out);
        const auto count = static_cast<std::size_t>(m) * static_cast<std::size_t>(n);
        if (out.size() != count) return 1;
        std::memcpy(c, out.data(), sizeof(float) * count);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

}  // extern "C"
