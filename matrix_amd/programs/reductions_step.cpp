// reductions_step.cpp -- the reductions workload as a compiled graph through the C++ graph API.
//
// X[256, 65536] float32 ~ N(0,1) (seed 0; in 30% of the rows the row maximum is copied to 1-3
// more positions, and the minimum likewise, to exercise first-index ties), held in 17 resident
// copies, one per reduction that reads X, so that no read of X in a step can be served by the
// 256 MB Infinity Cache from an earlier read of the same step (the executor runs independent
// reductions together, as group launches on two streams).
// The graph: Sum / Max / Min / ArgMax / ArgMin over axis 1 and over axis 0 of X; on
// X.reshape(64, 4, 4096, 16): Sum / Max / Min over axis 3 then axis 1, ArgMax / ArgMin over axis 3
// and over axis 1.  The j-th reduction that reads X reads copy j.  Built and compiled once, then
// executed `steps`
// times (execute + clear_trace_checks), as compile_metal / execute_metal do (Matrix.mm:8452-8475).
//
//   reductions_step [--steps K] [--warmup W]
// prints one JSON line: ms per step (wall clock around the timed steps, each ending in execute's
// stream wait), the step's algorithmic bytes (inputs read + outputs written) and GB/s.
#include "../host/matrix.hpp"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

int main(int argc, char** argv) {
    int steps = 20, warmup = 3;
    for (int i = 1; i + 1 < argc; i += 2) {
        if (!std::strcmp(argv[i], "--steps")) steps = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--warmup")) warmup = std::atoi(argv[i + 1]);
    }
    const size_m R = 256, Cc = 65536;
    try {
        std::vector<float> xv((size_t)R * Cc);
        std::mt19937_64 g(0);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        for (auto& v : xv) v = nd(g);
        std::uniform_real_distribution<double> u(0.0, 1.0);
        for (size_m r = 0; r < R; r++) {
            if (u(g) >= 0.3) continue;
            float* row = xv.data() + (size_t)r * Cc;
            float mx = row[0], mn = row[0];
            for (size_m j = 1; j < Cc; j++) { mx = row[j] > mx ? row[j] : mx; mn = row[j] < mn ? row[j] : mn; }
            const int k = 1 + (int)(u(g) * 3);
            for (int t = 0; t < k; t++) row[(size_t)(u(g) * Cc) % Cc] = mx;
            for (int t = 0; t < k; t++) row[(size_t)(u(g) * Cc) % Cc] = mn;
        }
        std::vector<matrix> X;
        for (int c = 0; c < 17; c++) X.push_back(matrix::from_host<float>({R, Cc}, xv));
        std::vector<matrix> outs;
        double bytes = 0;
        int j = 0;
        auto x = [&]() -> matrix& { return X[(j++) % X.size()]; };
        const double xb = (double)R * Cc * 4;
        for (int axis : {1, 0}) {
            const double ob = (axis == 1 ? R : Cc) * 4.0;
            outs.push_back(x().sum(axis)); outs.push_back(x().max(axis)); outs.push_back(x().min(axis));
            outs.push_back(x().argmax(axis)); outs.push_back(x().argmin(axis));
            bytes += 5 * (xb + ob);
        }
        const std::vector<size_m> r4 = {64, 4, 4096, 16};
        const double b3 = xb + xb / 16, b31 = xb / 16 + xb / 64;
        outs.push_back(x().reshape(r4).sum(3).sum(1));
        outs.push_back(x().reshape(r4).max(3).max(1));
        outs.push_back(x().reshape(r4).min(3).min(1));
        bytes += 3 * (b3 + b31);
        outs.push_back(x().reshape(r4).argmax(3)); outs.push_back(x().reshape(r4).argmax(1));
        outs.push_back(x().reshape(r4).argmin(3)); outs.push_back(x().reshape(r4).argmin(1));
        bytes += 2 * (b3 + xb + xb / 4);
        matrix::compile_gpu(outs);
        for (int i = 0; i < warmup; i++) {
            matrix::execute_gpu(outs);
            matrix::clear_trace_checks(outs);
        }
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; i++) {
            matrix::execute_gpu(outs);
            matrix::clear_trace_checks(outs);
        }
        auto t1 = std::chrono::steady_clock::now();
        const double ms = std::chrono::duration<double, std::milli>(t1 - t0).count() / (steps > 0 ? steps : 1);
        const char* env = std::getenv("MATRIX_AMD_STREAMS");
        std::printf("{\"workload\": \"reductions_step\", \"steps\": %d, \"warmup\": %d, \"ms_per_step\": %.4f, "
                    "\"step_bytes\": %.0f, \"GB/s\": %.1f, \"streams\": %d}\n",
                    steps, warmup, ms, bytes, bytes / (ms * 1e-3) / 1e9, env ? std::atoi(env) : 2);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "reductions_step: %s\n", e.what());
        return 1;
    }
    return 0;
}
