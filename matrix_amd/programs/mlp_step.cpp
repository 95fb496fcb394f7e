// mlp_step.cpp -- the compiled-graph MLP training step through the C++ graph API.
//
// 3-layer MLP 1024 -> 4096 -> 4096 -> 10, batch 512, float32: per layer
// h = max(x.dot(W) + b, 0) (no ReLU on the last), loss = ((y - t) * (y - t)).sum(); the
// gradient graph of the loss to every W and b comes from build_grad_graph.  The graph is built
// and compiled once, then executed `steps` times (execute + clear_trace_checks), as a caller of
// compile_metal / execute_metal does (Matrix.mm:8452-8475).  Inputs ~ N(0,1), weights
// ~ N(0, 1/fan_in), biases zero, targets ~ U(0,1), all seeded.
//
//   mlp_step [--steps K] [--warmup W] [--batch B] [--dump DIR]
// prints one JSON line: ms per step (wall clock around the timed steps, each step ending in
// the stream wait of execute), steps/s, the step's algorithmic TFLOP/s and the device
// allocations made during all the executes (0: compile allocated everything).  --dump writes the
// inputs, parameters, pre-activations, loss and gradients of the last step as raw float32 into DIR.
#include "../host/matrix.hpp"
#include "../../include/matrix_amd.h"

#include <chrono>
#include <fstream>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

static std::vector<float> normal(size_t n, uint64_t seed, float stddev) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> d(0.0f, stddev);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g);
    return v;
}

int main(int argc, char** argv) {
    int steps = 100, warmup = 5;
    size_m B = 512;
    std::string dump;
    for (int i = 1; i + 1 < argc; i += 2) {
        if (!std::strcmp(argv[i], "--steps")) steps = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--warmup")) warmup = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--batch")) B = (size_m)std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--dump")) dump = argv[i + 1];
    }
    const size_m D[4] = {1024, 4096, 4096, 10};
    try {
        matrix x = matrix::from_host<float>({B, D[0]}, normal((size_t)B * D[0], 1, 1.0f));
        std::vector<float> tv((size_t)B * D[3]);
        {
            std::mt19937_64 g(2);
            std::uniform_real_distribution<float> u(0.0f, 1.0f);
            for (auto& v : tv) v = u(g);
        }
        matrix t = matrix::from_host<float>({B, D[3]}, tv);
        std::vector<matrix> params;
        for (int l = 0; l < 3; l++) {
            params.push_back(matrix::from_host<float>({D[l], D[l + 1]},
                                                      normal((size_t)D[l] * D[l + 1], 10 + l, 1.0f / std::sqrt((float)D[l]))));
            params.push_back(matrix::zeros({D[l + 1]}));
        }
        matrix h = x;
        std::vector<matrix> zs;            // pre-activations, for --dump
        for (int l = 0; l < 3; l++) {
            matrix z = h.dot(params[2 * l]) + params[2 * l + 1];
            zs.push_back(z);
            h = l < 2 ? matrix::max(z, matrix::scalar(0.0f)) : z;
        }
        matrix d = h - t;
        matrix loss = (d * d).sum();
        std::vector<matrix> outs{loss};
        std::vector<matrix> grads = matrix::build_grad_graph(outs, params);
        std::vector<matrix> all = grads;
        all.push_back(loss);

        auto t0 = std::chrono::steady_clock::now();
        matrix::compile_gpu(all);
        auto t1 = std::chrono::steady_clock::now();
        uint64_t a0 = 0, f0 = 0, a1 = 0, f1 = 0;
        if (mx_hip_alloc_stats(&a0, &f0) != MX_OK) throw std::runtime_error(mx_last_error());
        for (int i = 0; i < warmup; i++) {
            matrix::execute_gpu(all);
            matrix::clear_trace_checks(all);
        }
        auto t2 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; i++) {
            matrix::execute_gpu(all);
            matrix::clear_trace_checks(all);
        }
        auto t3 = std::chrono::steady_clock::now();
        if (mx_hip_alloc_stats(&a1, &f1) != MX_OK) throw std::runtime_error(mx_last_error());
        if (!dump.empty()) {
            matrix::execute_gpu(all);      // one more step, whose values stay evaluated
            auto put = [&](const std::string& name, const matrix& m) {
                const std::vector<uint8_t> b = m.to_host_bytes();
                std::ofstream f(dump + "/" + name + ".bin", std::ios::binary);
                f.write(reinterpret_cast<const char*>(b.data()), (std::streamsize)b.size());
                if (!f) throw std::runtime_error("mlp_step: cannot write " + dump + "/" + name + ".bin");
            };
            put("x", x);
            put("t", t);
            for (int l = 0; l < 3; l++) {
                put("W" + std::to_string(l), params[2 * l]);
                put("b" + std::to_string(l), params[2 * l + 1]);
                put("gW" + std::to_string(l), grads[2 * l]);
                put("gb" + std::to_string(l), grads[2 * l + 1]);
                put("z" + std::to_string(l), zs[l]);
            }
            put("loss", loss);
        }
        const double ms = std::chrono::duration<double, std::milli>(t3 - t2).count() / (steps > 0 ? steps : 1);
        const double compile_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        // forward 2 B (D0 D1 + D1 D2 + D2 D3); backward twice that, less the input gradient of layer 1
        const double fwd = 2.0 * B * ((double)D[0] * D[1] + (double)D[1] * D[2] + (double)D[2] * D[3]);
        const double bwd = 2.0 * fwd - 2.0 * B * (double)D[0] * D[1];
        const double flop = fwd + bwd;
        const float lv = loss.to_host<float>()[0];
        std::printf("{\"workload\": \"mlp_step\", \"batch\": %u, \"steps\": %d, \"warmup\": %d, \"ms_per_step\": %.4f, "
                    "\"steps_per_s\": %.3f, \"tflops\": %.3f, \"flop_per_step\": %.0f, \"compile_ms\": %.2f, "
                    "\"loss\": %.6e, \"allocs_during_execute\": %llu, \"frees_during_execute\": %llu}\n",
                    B, steps, warmup, ms, 1000.0 / ms, flop / (ms * 1e-3) / 1e12, flop, compile_ms, (double)lv,
                    (unsigned long long)(a1 - a0), (unsigned long long)(f1 - f0));
    } catch (const std::exception& e) {
        std::fprintf(stderr, "mlp_step: %s\n", e.what());
        return 1;
    }
    return 0;
}
