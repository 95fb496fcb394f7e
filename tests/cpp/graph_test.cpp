// graph_test.cpp -- tests of the lazy-graph layer (matrix_amd/host/matrix.hpp).
//
//   graph_test cpu   graph building only (shape inference, errors, gradient-graph structure);
//                    touches no device
//   graph_test gpu   graphs evaluated on the GPU against double-precision host loops of the
//                    same mathematics (independent of the kernels and of the oracle)
//
// Prints "PASS <name>" / "FAIL <name>: <why>" per case; exit status 1 if any case failed.
#include "../../matrix_amd/host/matrix.hpp"
#include "../../include/matrix_amd.h"

#include <cmath>
#include <complex>
#include <cstdio>
#include <cstring>
#include <unordered_set>
#include <functional>
#include <random>
#include <string>
#include <vector>

static int g_fail = 0;

#define CASE(name) static void name()
#define EXPECT(cond, msg)                                                     \
    do {                                                                      \
        if (!(cond)) throw std::runtime_error(std::string(msg));              \
    } while (0)

static void run(const char* name, void (*fn)()) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception& e) {
        std::printf("FAIL %s: %s\n", name, e.what());
        g_fail++;
    }
    std::fflush(stdout);
}

template <typename F>
static bool throws(F&& f) {
    try { f(); } catch (const std::invalid_argument&) { return true; }
    return false;
}

static std::vector<float> randn(size_t n, uint64_t seed, float scale = 1.0f) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g) * scale;
    return v;
}
static std::vector<float> randu(size_t n, uint64_t seed, float lo, float hi) {
    std::mt19937_64 g(seed);
    std::uniform_real_distribution<float> d(lo, hi);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g);
    return v;
}

static double rel_err(const std::vector<float>& got, const std::vector<double>& ref) {
    double num = 0, den = 0;
    for (size_t i = 0; i < ref.size(); i++) {
        num += (got[i] - ref[i]) * (got[i] - ref[i]);
        den += ref[i] * ref[i];
    }
    return std::sqrt(num / (den > 0 ? den : 1));
}

// ------------------------------------------------------------------ CPU (build-only) cases
CASE(shapes_broadcast_and_reduce) {
    matrix a = matrix::leaf({4096, 1024});
    matrix b = matrix::leaf({1, 1024});
    matrix c = a + b;
    EXPECT(c.dims == 2 && c.shape()[0] == 4096 && c.shape()[1] == 1024, "broadcast shape");
    matrix s = c.sum(1);
    EXPECT(s.dims == 1 && s.shape()[0] == 4096, "sum(1) shape");
    EXPECT(c.sum(1, true).dims == 2 && c.sum(1, true).shape()[1] == 1, "keepdims shape");
    matrix g = c.sum();
    EXPECT(g.dims == 0 && g.total_size() == 1, "global sum is rank 0");
    EXPECT(c.argmax(0).type == dtype::Int32 && c.argmax(0).shape()[0] == 1024, "argmax dtype / shape");
    EXPECT(throws([&] { (void)(matrix::leaf({3, 4}) + matrix::leaf({5, 4})); }), "incompatible broadcast throws");
    EXPECT(throws([&] { (void)a.sum(2); }), "axis out of range throws");
}

CASE(shapes_dot_and_conv) {
    matrix a = matrix::leaf({16, 64, 32});
    matrix b = matrix::leaf({32, 48});
    matrix c = a.dot(b);
    EXPECT(c.dims == 3 && c.shape()[0] == 16 && c.shape()[1] == 64 && c.shape()[2] == 48, "dot shape");
    EXPECT(throws([&] { (void)a.dot(matrix::leaf({31, 48})); }), "core-dimension mismatch throws");
    // a float B in its [K, N] layout reaches the GEMM as the transposed view of its own storage
    EXPECT(c.tape && c.tape->input_at(1).storage == b.storage, "fp32 N-major B is not copied");
    for (dtype t : {dtype::Float16, dtype::BFloat16}) {
        matrix b16 = matrix::leaf({32, 48}, t);
        matrix c16 = matrix::leaf({64, 32}, t).dot(b16);
        EXPECT(c16.tape->input_at(1).storage == b16.storage, "16-bit N-major B is not copied");
        matrix c40 = matrix::leaf({64, 32}, t).dot(matrix::leaf({32, 44}, t));
        EXPECT(c40.tape->input_at(1).is_contiguous(), "16-bit N not a multiple of 8: B^T is packed");
        // the vjp's g^T . A: g^T is an M-major view of g, read without a copy
        matrix g16 = matrix::leaf({64, 48}, t);
        matrix gt = g16.transpose({1, 0}).dot(matrix::leaf({64, 32}, t));
        EXPECT(gt.tape->input_at(0).storage == g16.storage, "16-bit M-major A is not copied");
        matrix gt44 = matrix::leaf({64, 44}, t).transpose({1, 0}).dot(matrix::leaf({64, 32}, t));
        EXPECT(gt44.tape->input_at(0).is_contiguous(), "16-bit M not a multiple of 8: A is packed");
    }
    matrix g32 = matrix::leaf({64, 48});
    EXPECT(g32.transpose({1, 0}).dot(matrix::leaf({64, 32})).tape->input_at(0).storage == g32.storage,
           "fp32 M-major A is not copied");
    EXPECT(matrix::leaf({64, 42}).transpose({1, 0}).dot(matrix::leaf({64, 32})).tape->input_at(0).is_contiguous(),
           "fp32 M not a multiple of 4: A is packed");
    matrix bs = matrix::leaf({32, 48});
    EXPECT(matrix::leaf({8, 1, 32}).dot(bs).tape->input_at(1).storage == bs.storage,
           "fp32, at most 16 rows of A (the streaming kernel's N-major form): B is not copied");
    matrix c10 = a.dot(matrix::leaf({32, 10}));
    EXPECT(c10.tape->input_at(1).is_contiguous(), "N not a multiple of 4: B^T is packed");
    matrix x = matrix::leaf({2, 56, 56, 64});
    matrix w = matrix::leaf({128, 3, 3, 64});
    matrix y = matrix::conv2d(x, w, 1, 1, 1, 1);
    EXPECT(y.shape()[0] == 2 && y.shape()[1] == 56 && y.shape()[2] == 56 && y.shape()[3] == 128, "conv2d shape");
    matrix y2 = matrix::conv2d(x, matrix::leaf({32, 1, 1, 64}), 2, 2);
    EXPECT(y2.shape()[1] == 28 && y2.shape()[2] == 28, "strided 1x1 shape");
    EXPECT(throws([&] { (void)matrix::conv2d(x, matrix::leaf({8, 3, 3, 60})); }), "channel mismatch throws");
}

CASE(views_share_storage) {
    matrix a = matrix::leaf({3, 4, 5});
    matrix t = a.transpose({2, 0, 1});
    EXPECT(t.storage == a.storage && t.shape()[0] == 5 && t.strides()[0] == 1 && !t.is_contiguous(), "transpose view");
    matrix r = a.reshape({12, 5});
    EXPECT(r.storage == a.storage && r.is_contiguous(), "reshape of contiguous is a view");
    matrix rt = t.reshape({5, 12});
    EXPECT(rt.storage != a.storage, "reshape of a strided view copies");
    matrix bb = matrix::leaf({1, 5}).broadcast_to({4, 5});
    EXPECT(bb.strides()[0] == 0, "broadcast stride 0");
}

CASE(grad_graph_structure) {
    matrix x = matrix::leaf({8, 16});
    matrix w = matrix::leaf({16, 4});
    matrix b = matrix::leaf({4});
    matrix y = matrix::max(x.dot(w) + b, matrix::scalar(0.0f));
    matrix loss = (y * y).sum();
    std::vector<matrix> outs{loss}, params{w, b};
    std::vector<matrix> g = matrix::build_grad_graph(outs, params);
    EXPECT(g.size() == 2, "two gradients");
    EXPECT(g[0].dims == 2 && g[0].shape()[0] == 16 && g[0].shape()[1] == 4, "dW shape");
    EXPECT(g[1].dims == 1 && g[1].shape()[0] == 4, "db shape (unbroadcast)");
    matrix unused = matrix::leaf({3});
    std::vector<matrix> p2{unused};
    std::vector<matrix> g2 = matrix::build_grad_graph(outs, p2);
    EXPECT(g2[0].tape == nullptr && g2[0].shape()[0] == 3, "unused parameter gets zeros");
    EXPECT(throws([&] { (void)matrix::value_and_grad([](std::vector<matrix> p) { return p[0] * 2.0f; })({matrix::leaf({3})}); }),
           "value_and_grad needs a single-element output");
    // the vjp of Max: one MaxGrad node per operand when the incoming gradient is a contiguous node
    // output of the broadcast's shape ((y * y).sum() gives 2 y g), the four-node form (with its
    // Equal) when it is not (the gradient of z.sum(1) is a stride-0 broadcast view)
    auto has = [](const matrix& m, const char* name) {
        std::unordered_set<const Primitive*> seen;
        std::function<bool(const matrix&)> walk = [&](const matrix& n) -> bool {
            if (!n.tape || !seen.insert(n.tape.get()).second) return false;
            if (std::string(n.tape->name()) == name) return true;
            for (uint32_t i = 0; i < n.tape->num_inputs(); i++)
                if (walk(n.tape->input_at(i))) return true;
            return false;
        };
        return walk(m);
    };
    EXPECT(has(g[0], "MaxGrad") && !has(g[0], "Equal"), "dense layer: fused Max backward");
    matrix z = matrix::max(x, matrix::scalar(0.0f));
    std::vector<matrix> outs3{z.sum(1).sum()}, p3{x};
    std::vector<matrix> g3 = matrix::build_grad_graph(outs3, p3);
    EXPECT(!has(g3[0], "MaxGrad") && has(g3[0], "Equal"), "broadcast gradient: four-node Max backward");
}

// ------------------------------------------------------------------ GPU cases
CASE(gpu_add_then_rowsum) {
    const size_m R = 4096, Cc = 1024;
    auto av = randn((size_t)R * Cc, 0);
    auto bv = randu(Cc, 1, -1.f, 1.f);
    matrix a = matrix::from_host<float>({R, Cc}, av);
    matrix b = matrix::from_host<float>({1, Cc}, bv);
    matrix c = a + b;
    matrix s = c.sum(1);
    std::vector<matrix> outs{c, s};
    matrix::eval(outs);
    auto cg = c.to_host<float>();
    auto sg = s.to_host<float>();
    for (size_t i = 0; i < (size_t)R * Cc; i++)
        EXPECT(cg[i] == av[i] + bv[i % Cc], "add is not exact");
    for (size_t r = 0; r < R; r++) {
        double ref = 0, mag = 0;
        for (size_t j = 0; j < Cc; j++) { ref += (double)cg[r * Cc + j]; mag += std::fabs(cg[r * Cc + j]); }
        EXPECT(std::fabs(sg[r] - ref) <= 1e-4 * mag, "row sum beyond 1e-4 of sum|x|");
    }
}

// A reduction over a broadcast node's last axis is fused into that node's launch: the results
// stay right when the graph is re-executed after a leaf changes, when a second reduction of the
// same node is added (not fused), when only the reduction is executed, and when a reduction is
// attached to a node that has already run.
CASE(gpu_fused_reduction_lifecycle) {
    const size_m R = 512, Cc = 768;
    auto av = randn((size_t)R * Cc, 20);
    auto bv = randu(Cc, 21, -1.f, 1.f);
    matrix a = matrix::from_host<float>({R, Cc}, av);
    matrix b = matrix::from_host<float>({1, Cc}, bv);
    matrix c = a * b;
    matrix s = c.sum(1);                       // fused into c
    matrix m = c.max(1);                       // second reduction of c: its own launch
    std::vector<matrix> outs{c, s, m};
    auto check = [&](const std::vector<float>& aa, const char* when) {
        auto cg = c.to_host<float>();
        auto sg = s.to_host<float>();
        auto mg = m.to_host<float>();
        for (size_t r = 0; r < R; r++) {
            double ref = 0, mag = 0;
            float mx = -3.4028234663852886e38f;
            for (size_t j = 0; j < Cc; j++) {
                const float v = aa[r * Cc + j] * bv[j];
                EXPECT(cg[r * Cc + j] == v, std::string("product not exact ") + when);
                ref += v; mag += std::fabs(v);
                if (mx < v) mx = v;
            }
            EXPECT(std::fabs(sg[r] - ref) <= 1e-4 * mag, std::string("fused row sum ") + when);
            EXPECT(mg[r] == mx, std::string("row max ") + when);
        }
    };
    matrix::compile_gpu(outs);
    matrix::execute_gpu(outs);
    check(av, "first run");
    for (int it = 0; it < 2; it++) {           // new leaf values, re-executed
        auto av2 = randn((size_t)R * Cc, 30 + it);
        std::memcpy(a.host_data(), av2.data(), av2.size() * sizeof(float));
        a.mark_changed();
        matrix::clear_trace_checks(outs);
        matrix::execute_gpu(outs);
        check(av2, "after mark_changed");
        av = av2;
    }
    std::vector<matrix> only_s{s};             // only the reduction: the producer runs (fused) first
    matrix::clear_trace_checks(only_s);
    matrix::execute_gpu(only_s);
    check(av, "executing the reduction alone");
    matrix s2 = c.sum(1);                       // attached after c ran: computed by its own launch
    std::vector<matrix> late{s2};
    matrix::eval(late);
    auto s2g = s2.to_host<float>();
    auto sg = s.to_host<float>();
    for (size_t r = 0; r < R; r++) {
        double mag = 0;
        for (size_t j = 0; j < Cc; j++) mag += std::fabs(av[r * Cc + j] * bv[j]);
        EXPECT(std::fabs(s2g[r] - sg[r]) <= 2e-4 * mag, "late reduction");
    }
    // the producer alone while its fused reduction stays evaluated (a boundary of this execute):
    // the product is recomputed by the plain broadcast launch and the reduction keeps its values
    auto av3 = randn((size_t)R * Cc, 50);
    std::memcpy(a.host_data(), av3.data(), av3.size() * sizeof(float));
    a.mark_changed();
    std::vector<matrix> only_c{c};
    matrix::clear_trace_checks(only_c);
    matrix::execute_gpu(only_c);
    auto cg3 = c.to_host<float>();
    for (size_t i = 0; i < (size_t)R * Cc; i++) EXPECT(cg3[i] == av3[i] * bv[i % Cc], "product recomputed alone");
    auto sg3 = s.to_host<float>();
    EXPECT(std::memcmp(sg3.data(), sg.data(), sg.size() * sizeof(float)) == 0,
           "an evaluated fused reduction was rewritten by its producer");
}

// A dense layer's bias + ReLU, h = max(x . W + b, 0): the Dot launches the product, the bias Add
// and the Max together (mx_launch_batched_matmul_bias_act).  t, z and h must hold the product,
// z = t + b and h = max(z, 0) exactly (from the downloaded t), on the first run, after the bias
// and x change on the host, and when only h is executed.
CASE(gpu_dense_bias_relu_lifecycle) {
    const size_m R = 64, K = 96, N = 256;
    auto xv = randn((size_t)R * K, 40);
    auto wv = randn((size_t)K * N, 41);
    auto bv = randu(N, 42, -1.f, 1.f);
    matrix x = matrix::from_host<float>({R, K}, xv);
    matrix W = matrix::from_host<float>({K, N}, wv);
    matrix b = matrix::from_host<float>({N}, bv);
    matrix t = x.dot(W);
    matrix z = t + b;
    matrix h = matrix::max(z, matrix::scalar(0.0f));
    std::vector<matrix> outs{t, z, h};
    auto check = [&](const std::vector<float>& xx, const std::vector<float>& bb, const char* when) {
        auto tg = t.to_host<float>();
        auto zg = z.to_host<float>();
        auto hg = h.to_host<float>();
        size_t clamped = 0;
        for (size_t r = 0; r < R; r++)
            for (size_t j = 0; j < N; j++) {
                double ref = 0, mag = 0;
                for (size_t k = 0; k < K; k++) {
                    ref += (double)xx[r * K + k] * wv[k * N + j];
                    mag += std::fabs((double)xx[r * K + k] * wv[k * N + j]);
                }
                const size_t i = r * N + j;
                EXPECT(std::fabs(tg[i] - ref) <= 1e-5 * mag + 1e-6, std::string("product ") + when);
                const float zr = tg[i] + bb[j];
                EXPECT(zg[i] == zr, std::string("bias add ") + when);
                EXPECT(hg[i] == ((zr < 0.0f) ? 0.0f : zr), std::string("relu ") + when);
                clamped += hg[i] != zg[i];
            }
        EXPECT(clamped > 0 && clamped < (size_t)R * N, std::string("relu clamps some ") + when);
    };
    matrix::compile_gpu(outs);
    matrix::execute_gpu(outs);
    check(xv, bv, "first run");
    auto bv2 = randu(N, 43, -2.f, 2.f);            // new bias: z and h must follow it
    std::memcpy(b.host_data(), bv2.data(), bv2.size() * sizeof(float));
    b.mark_changed();
    matrix::clear_trace_checks(outs);
    matrix::execute_gpu(outs);
    check(xv, bv2, "after the bias changed");
    auto xv2 = randn((size_t)R * K, 44);          // new input, only h requested
    std::memcpy(x.host_data(), xv2.data(), xv2.size() * sizeof(float));
    x.mark_changed();
    std::vector<matrix> only_h{h};
    matrix::clear_trace_checks(only_h);
    matrix::execute_gpu(only_h);
    check(xv2, bv2, "executing h alone");
    // the product alone while z and h stay evaluated: the Dot runs without its epilogue, z and h
    // keep their values
    const auto zg0 = z.to_host<float>(), hg0 = h.to_host<float>();
    auto xv3 = randn((size_t)R * K, 45);
    std::memcpy(x.host_data(), xv3.data(), xv3.size() * sizeof(float));
    x.mark_changed();
    std::vector<matrix> only_t{t};
    matrix::clear_trace_checks(only_t);
    matrix::execute_gpu(only_t);
    EXPECT(z.to_host<float>() == zg0 && h.to_host<float>() == hg0, "an evaluated epilogue was rewritten by the Dot");
    auto tg3 = t.to_host<float>();
    for (size_t r = 0; r < R; r++)
        for (size_t j = 0; j < N; j++) {
            double ref = 0, mag = 0;
            for (size_t k = 0; k < K; k++) {
                ref += (double)xv3[r * K + k] * wv[k * N + j];
                mag += std::fabs((double)xv3[r * K + k] * wv[k * N + j]);
            }
            EXPECT(std::fabs(tg3[r * N + j] - ref) <= 1e-5 * mag + 1e-6, "product recomputed alone");
        }
}

// Independent reductions with one descriptor run as group launches (horizontal fusion): five over
// axis 1, three over axis 0, two over axis 3 of a reshape and the two chained over axis 1 after
// them.  d reduces with the axis-0 descriptor but depends on one of that group's members, so it
// must run after the group, not in it.  Every output equals host loops, also when executed again
// after a leaf changes.
CASE(gpu_grouped_reductions) {
    const size_m R = 96, Cc = 4096;
    std::vector<std::vector<float>> xv;
    std::vector<matrix> x;
    for (int k = 0; k < 4; k++) {
        auto v = randn((size_t)R * Cc, 40 + k);
        for (size_t r = 0; r < R; r += 3) v[r * Cc + 7] = v[r * Cc + 900] = 5.0f;   // ties of the row maxima
        xv.push_back(v);
        x.push_back(matrix::from_host<float>({R, Cc}, v));
    }
    const std::vector<size_m> r4 = {R, 4, 64, 16};
    matrix a_max0 = x[1].max(0);
    matrix d = (x[0] + a_max0.unsqueeze(0)).max(0);
    std::vector<matrix> outs{x[0].sum(1), x[1].max(1), x[2].min(1), x[3].argmax(1), x[0].argmin(1),
                             x[1].sum(0), a_max0, x[3].argmin(0), d,
                             x[2].reshape(r4).sum(3).sum(1), x[3].reshape(r4).max(3).max(1)};
    auto check = [&](const char* when) {
        auto at = [&](int k, size_t r, size_t c) { return xv[k][r * Cc + c]; };
        // axis 1
        auto s1 = outs[0].to_host<float>(); auto m1 = outs[1].to_host<float>(); auto n1 = outs[2].to_host<float>();
        auto am1 = outs[3].to_host<int32_t>(); auto an1 = outs[4].to_host<int32_t>();
        for (size_t r = 0; r < R; r++) {
            double s = 0, mag = 0;
            float mx = -3.4028234663852886e38f, mn = 3.4028234663852886e38f, amv = mx, anv = mn;
            int32_t ia = 0, in_ = 0;
            for (size_t c = 0; c < Cc; c++) {
                s += at(0, r, c); mag += std::fabs(at(0, r, c));
                if (mx < at(1, r, c)) mx = at(1, r, c);
                if (at(2, r, c) < mn) mn = at(2, r, c);
                if (at(3, r, c) > amv) { amv = at(3, r, c); ia = (int32_t)c; }
                if (at(0, r, c) < anv) { anv = at(0, r, c); in_ = (int32_t)c; }
            }
            EXPECT(std::fabs(s1[r] - s) <= 1e-4 * mag, std::string("axis-1 sum ") + when);
            EXPECT(m1[r] == mx && n1[r] == mn, std::string("axis-1 max / min ") + when);
            EXPECT(am1[r] == ia && an1[r] == in_, std::string("axis-1 argmax / argmin ") + when);
        }
        // axis 0, and d = max over rows of x0 + max0(x1)
        auto s0 = outs[5].to_host<float>(); auto m0 = outs[6].to_host<float>();
        auto an0 = outs[7].to_host<int32_t>(); auto dg = outs[8].to_host<float>();
        for (size_t c = 0; c < Cc; c++) {
            double s = 0, mag = 0;
            float mx = -3.4028234663852886e38f, anv = 3.4028234663852886e38f;
            int32_t in_ = 0;
            for (size_t r = 0; r < R; r++) {
                s += at(1, r, c); mag += std::fabs(at(1, r, c));
                if (mx < at(1, r, c)) mx = at(1, r, c);
                if (at(3, r, c) < anv) { anv = at(3, r, c); in_ = (int32_t)r; }
            }
            float dm = -3.4028234663852886e38f;
            for (size_t r = 0; r < R; r++) { const float v = at(0, r, c) + mx; if (dm < v) dm = v; }
            EXPECT(std::fabs(s0[c] - s) <= 1e-4 * mag, std::string("axis-0 sum ") + when);
            EXPECT(m0[c] == mx && an0[c] == in_, std::string("axis-0 max / argmin ") + when);
            EXPECT(dg[c] == dm, std::string("dependent reduction ") + when);
        }
        // chains over the reshape [R, 4, 64, 16]: axis 3, then axis 1
        auto cs = outs[9].to_host<float>(); auto cm = outs[10].to_host<float>();
        for (size_t r = 0; r < R; r++)
            for (size_t j = 0; j < 64; j++) {
                double s = 0, mag = 0;
                float mx = -3.4028234663852886e38f;
                for (size_t q = 0; q < 4; q++) {
                    float m3 = -3.4028234663852886e38f;
                    for (size_t t = 0; t < 16; t++) {
                        const size_t c = q * 1024 + j * 16 + t;
                        s += at(2, r, c); mag += std::fabs(at(2, r, c));
                        if (m3 < at(3, r, c)) m3 = at(3, r, c);
                    }
                    if (mx < m3) mx = m3;
                }
                EXPECT(std::fabs(cs[r * 64 + j] - s) <= 1e-4 * mag, std::string("chained sum ") + when);
                EXPECT(cm[r * 64 + j] == mx, std::string("chained max ") + when);
            }
    };
    matrix::compile_gpu(outs);
    matrix::execute_gpu(outs);
    check("first run");
    auto v2 = randn((size_t)R * Cc, 50);
    std::memcpy(x[3].host_data(), v2.data(), v2.size() * sizeof(float));
    xv[3] = v2;
    x[3].mark_changed();
    matrix::clear_trace_checks(outs);
    matrix::execute_gpu(outs);
    check("after mark_changed");
}

CASE(gpu_reductions_and_views) {
    const size_m R = 64, Cc = 4 * 256 * 16;
    auto xv = randn((size_t)R * Cc, 2);
    matrix x = matrix::from_host<float>({R, Cc}, xv);
    matrix mx0 = x.max(0), mn1 = x.min(1), am1 = x.argmax(1), an0 = x.argmin(0);
    matrix chain = x.reshape({16, 4, 256, 64}).sum(3).sum(1);     // reduce a strided split
    matrix tsum = x.transpose({1, 0}).sum(1);                      // reduce over a transposed view
    std::vector<matrix> outs{mx0, mn1, am1, an0, chain, tsum};
    matrix::eval(outs);
    auto a0 = mx0.to_host<float>(), a1 = mn1.to_host<float>(), t1 = tsum.to_host<float>(), ch = chain.to_host<float>();
    auto i1 = am1.to_host<int32_t>(), i0 = an0.to_host<int32_t>();
    for (size_t j = 0; j < Cc; j++) {
        float m = -3.4028234663852886e38f, mn = 3.4028234663852886e38f;
        int32_t im = 0;
        double s = 0;
        for (size_t r = 0; r < R; r++) {
            const float v = xv[r * Cc + j];
            if (m < v) m = v;
            if (v < mn) { mn = v; im = (int32_t)r; }
            s += v;
        }
        EXPECT(a0[j] == m, "max(0)");
        EXPECT(i0[j] == im, "argmin(0)");
        EXPECT(std::fabs(t1[j] - s) <= 1e-4 * R * 4, "sum over transposed view");
    }
    for (size_t r = 0; r < R; r++) {
        float mn = 3.4028234663852886e38f, mx = -3.4028234663852886e38f;
        int32_t im = 0;
        for (size_t j = 0; j < Cc; j++) {
            const float v = xv[r * Cc + j];
            if (v < mn) mn = v;
            if (v > mx) { mx = v; im = (int32_t)j; }
        }
        EXPECT(a1[r] == mn, "min(1)");
        EXPECT(i1[r] == im, "argmax(1)");
    }
    // chain: [16,4,256,64] summed over axes 3 then 1 -> [16,256]
    for (size_t a = 0; a < 16; a++)
        for (size_t c = 0; c < 256; c++) {
            double s = 0, mag = 0;
            for (size_t b = 0; b < 4; b++)
                for (size_t d = 0; d < 64; d++) {
                    const float v = xv[((a * 4 + b) * 256 + c) * 64 + d];
                    s += v;
                    mag += std::fabs(v);
                }
            EXPECT(std::fabs(ch[a * 256 + c] - s) <= 1e-4 * mag, "sum(3).sum(1) chain");
        }
}

CASE(gpu_dot_batched_broadcast) {
    const size_m B = 4, M = 200, K = 300, N = 150;
    auto av = randn((size_t)B * M * K, 3, 1.0f / std::sqrt((float)K));
    auto bv = randn((size_t)K * N, 4);
    matrix a = matrix::from_host<float>({B, M, K}, av);
    matrix b = matrix::from_host<float>({K, N}, bv);
    matrix c = a.dot(b);
    auto cg = c.to_host<float>();
    std::vector<double> ref((size_t)B * M * N, 0.0);
    for (size_t bb = 0; bb < B; bb++)
        for (size_t m = 0; m < M; m++)
            for (size_t k = 0; k < K; k++) {
                const double x = av[(bb * M + m) * K + k];
                for (size_t n = 0; n < N; n++) ref[(bb * M + m) * N + n] += x * bv[k * N + n];
            }
    EXPECT(rel_err(cg, ref) <= 1e-4, "dot normwise error above 1e-4");
}

CASE(gpu_conv2d_nchw_views) {
    const size_m N = 2, C = 16, H = 9, W = 8, O = 12;
    auto xv = randn((size_t)N * C * H * W, 5);
    auto wv = randn((size_t)O * C * 9, 6, 0.2f);
    matrix x = matrix::from_host<float>({N, C, H, W}, xv).transpose({0, 2, 3, 1});   // NHWC view
    matrix w = matrix::from_host<float>({O, C, 3, 3}, wv).transpose({0, 2, 3, 1});   // OHWI view
    matrix y = matrix::conv2d(x, w, 1, 1, 1, 1);
    auto yg = y.to_host<float>();
    std::vector<double> ref((size_t)N * H * W * O, 0.0);
    for (size_t n = 0; n < N; n++)
        for (size_t oh = 0; oh < H; oh++)
            for (size_t ow = 0; ow < W; ow++)
                for (size_t o = 0; o < O; o++) {
                    double s = 0;
                    for (int kh = 0; kh < 3; kh++)
                        for (int kw = 0; kw < 3; kw++) {
                            const int ih = (int)oh - 1 + kh, iw = (int)ow - 1 + kw;
                            if (ih < 0 || iw < 0 || ih >= (int)H || iw >= (int)W) continue;
                            for (size_t c = 0; c < C; c++)
                                s += (double)xv[((n * C + c) * H + ih) * W + iw] * wv[((o * C + c) * 3 + kh) * 3 + kw];
                        }
                    ref[((n * H + oh) * W + ow) * O + o] = s;
                }
    EXPECT(rel_err(yg, ref) <= 1e-4, "conv2d normwise error above 1e-4");
}

// A small MLP training step: forward loss and every parameter gradient against a
// double-precision host forward / backward of the same network.
struct HostMLP {
    size_m B, D0, D1, D2, D3;
};

static void host_mlp(const HostMLP& s, const std::vector<float>& x, const std::vector<float>& t,
                     const std::vector<std::vector<float>>& W, const std::vector<std::vector<float>>& b, double& loss,
                     std::vector<std::vector<double>>& dW, std::vector<std::vector<double>>& db) {
    const size_m dimsv[4] = {s.D0, s.D1, s.D2, s.D3};
    std::vector<std::vector<double>> act(4), pre(4);
    act[0].assign(x.begin(), x.end());
    for (int l = 0; l < 3; l++) {
        const size_m din = dimsv[l], dout = dimsv[l + 1];
        pre[l + 1].assign((size_t)s.B * dout, 0.0);
        for (size_t i = 0; i < s.B; i++)
            for (size_t k = 0; k < din; k++) {
                const double a = act[l][i * din + k];
                for (size_t j = 0; j < dout; j++) pre[l + 1][i * dout + j] += a * W[l][k * dout + j];
            }
        act[l + 1].resize(pre[l + 1].size());
        for (size_t i = 0; i < s.B; i++)
            for (size_t j = 0; j < dout; j++) {
                const double v = pre[l + 1][i * dout + j] + b[l][j];
                pre[l + 1][i * dout + j] = v;
                act[l + 1][i * dout + j] = l < 2 ? (v > 0 ? v : 0) : v;
            }
    }
    loss = 0;
    std::vector<double> g((size_t)s.B * s.D3);
    for (size_t i = 0; i < g.size(); i++) {
        const double d = act[3][i] - t[i];
        loss += d * d;
        g[i] = 2 * d;
    }
    dW.assign(3, {});
    db.assign(3, {});
    for (int l = 2; l >= 0; --l) {
        const size_m din = dimsv[l], dout = dimsv[l + 1];
        if (l < 2)
            for (size_t i = 0; i < g.size(); i++) g[i] = pre[l + 1][i] > 0 ? g[i] : 0.0;   // ReLU (tie at 0 -> 0)
        dW[l].assign((size_t)din * dout, 0.0);
        db[l].assign(dout, 0.0);
        for (size_t i = 0; i < s.B; i++)
            for (size_t j = 0; j < dout; j++) {
                const double gv = g[i * dout + j];
                db[l][j] += gv;
                for (size_t k = 0; k < din; k++) dW[l][k * dout + j] += act[l][i * din + k] * gv;
            }
        std::vector<double> gin((size_t)s.B * din, 0.0);
        for (size_t i = 0; i < s.B; i++)
            for (size_t k = 0; k < din; k++) {
                double acc = 0;
                for (size_t j = 0; j < dout; j++) acc += g[i * dout + j] * W[l][k * dout + j];
                gin[i * din + k] = acc;
            }
        g.swap(gin);
    }
}

CASE(gpu_mlp_training_step_compile_once) {
    const HostMLP s{32, 64, 96, 80, 10};
    const size_m dimsv[4] = {s.D0, s.D1, s.D2, s.D3};
    auto xv = randn((size_t)s.B * s.D0, 7);
    auto tv = randu((size_t)s.B * s.D3, 8, 0.f, 1.f);
    std::vector<std::vector<float>> Wv(3), bv(3);
    for (int l = 0; l < 3; l++) {
        Wv[l] = randn((size_t)dimsv[l] * dimsv[l + 1], 10 + l, 1.0f / std::sqrt((float)dimsv[l]));
        bv[l] = randn(dimsv[l + 1], 20 + l, 0.1f);
    }
    matrix x = matrix::from_host<float>({s.B, s.D0}, xv);
    matrix t = matrix::from_host<float>({s.B, s.D3}, tv);
    std::vector<matrix> params;
    for (int l = 0; l < 3; l++) {
        params.push_back(matrix::from_host<float>({dimsv[l], dimsv[l + 1]}, Wv[l]));
        params.push_back(matrix::from_host<float>({dimsv[l + 1]}, bv[l]));
    }
    matrix h1 = matrix::max(x.dot(params[0]) + params[1], matrix::scalar(0.0f));
    matrix h2 = matrix::max(h1.dot(params[2]) + params[3], matrix::scalar(0.0f));
    matrix y = h2.dot(params[4]) + params[5];
    matrix loss = ((y - t) * (y - t)).sum();
    std::vector<matrix> outs{loss};
    std::vector<matrix> grads = matrix::build_grad_graph(outs, params);
    std::vector<matrix> all = grads;
    all.push_back(loss);
    matrix::compile_gpu(all);
    // five executes of the compiled graph; new inputs before executes 2 and 4 (host write +
    // mark_changed); no execute allocates device memory (an execute may free: the executor's
    // cache of recent schedules drops the oldest, and with it the earlier cases' graphs)
    uint64_t a0 = 0, f0 = 0, a1 = 0, f1 = 0;
    EXPECT(mx_hip_alloc_stats(&a0, &f0) == MX_OK, "alloc stats");
    for (int iter = 0; iter < 5; iter++) {
        if (iter == 2 || iter == 4) {
            auto x2 = randn((size_t)s.B * s.D0, 99 + iter);
            std::memcpy(x.host_data(), x2.data(), x2.size() * 4);
            x.mark_changed();
            xv = x2;
        }
        matrix::execute_gpu(all);
        EXPECT(mx_hip_alloc_stats(&a1, &f1) == MX_OK && a1 == a0,
               "execute " + std::to_string(iter) + " allocated device memory: " + std::to_string(a1 - a0) +
                   " allocations");
        double lref;
        std::vector<std::vector<double>> dW, db;
        host_mlp(s, xv, tv, Wv, bv, lref, dW, db);
        const float lg = loss.to_host<float>()[0];
        EXPECT(std::fabs(lg - lref) <= 1e-4 * std::fabs(lref), "loss mismatch");
        for (int l = 0; l < 3; l++) {
            EXPECT(rel_err(grads[2 * l].to_host<float>(), dW[l]) <= 1e-4, "dW mismatch, layer " + std::to_string(l));
            EXPECT(rel_err(grads[2 * l + 1].to_host<float>(), db[l]) <= 1e-4, "db mismatch, layer " + std::to_string(l));
        }
        EXPECT(mx_hip_alloc_stats(&a1, &f1) == MX_OK && a1 == a0,
               "reading the results of execute " + std::to_string(iter) + " allocated device memory: " +
                   std::to_string(a1 - a0) + " allocations");
        matrix::clear_trace_checks(all);
    }
}

CASE(gpu_value_and_grad) {
    auto xv = randn(100, 30);
    matrix x = matrix::from_host<float>({100}, xv);
    auto [val, g] = matrix::value_and_grad([](std::vector<matrix> p) { return (p[0] * p[0] * 3.0f).sum(); })({x});
    double ref = 0;
    for (float v : xv) ref += 3.0 * v * v;
    EXPECT(std::fabs(val.to_host<float>()[0] - ref) <= 1e-4 * ref, "value");
    auto gv = g[0].to_host<float>();
    std::vector<double> gref(xv.size());
    for (size_t i = 0; i < xv.size(); i++) gref[i] = 6.0 * xv[i];
    EXPECT(rel_err(gv, gref) <= 1e-6, "gradient of 3 x^2");
    // gradients through Max against a scalar: x.max(0.5).sum(1).sum() takes the four-node vjp (the
    // gradient reaching the Max is a broadcast view), (m * m).sum() the fused one; ties (x == 0.5)
    // send the gradient to the scalar, so x gets 0 there
    auto xv2 = randn(8 * 16, 31);
    for (size_t i = 0; i < xv2.size(); i += 7) xv2[i] = 0.5f;
    matrix x2 = matrix::from_host<float>({8, 16}, xv2);
    auto [v1, g1] = matrix::value_and_grad([](std::vector<matrix> p) {
        return matrix::max(p[0], matrix::scalar(0.5f)).sum(1).sum();
    })({x2});
    auto [v2, g2] = matrix::value_and_grad([](std::vector<matrix> p) {
        matrix m = matrix::max(p[0], matrix::scalar(0.5f));
        return (m * m).sum();
    })({x2});
    auto g1v = g1[0].to_host<float>();
    auto g2v = g2[0].to_host<float>();
    for (size_t i = 0; i < xv2.size(); i++) {
        const float m = xv2[i] < 0.5f ? 0.5f : xv2[i];
        const bool to_x = xv2[i] > 0.5f;
        EXPECT(g1v[i] == (to_x ? 1.0f : 0.0f), "max gradient, four-node form");
        EXPECT(g2v[i] == (to_x ? 2.0f * m : 0.0f), "max gradient, fused form");
    }
}

// complex64 (type code 9): Add / Sub / Mul / Divide build and promote real operands (a real leaf
// next to a complex one is cast to complex64); the ops the reference has no complex64 path for
// (max / min / equal, the reductions, dot, conv, a cast back to a real dtype) throw at construction.
template <typename F>
static bool throws_runtime(F&& f) {
    try { f(); } catch (const std::runtime_error&) { return true; }
    return false;
}

CASE(complex_construction_rules) {
    using cf = std::complex<float>;
    matrix z = matrix::from_host<cf>({4, 3}, std::vector<cf>(12, cf(1.0f, 2.0f)));
    matrix r = matrix::from_host<float>({3}, std::vector<float>(3, 0.5f));
    EXPECT(z.type == dtype::Complex64, "std::complex<float> leaf is not Complex64");
    matrix p = z * r;
    EXPECT(p.type == dtype::Complex64 && p.shape_vec() == std::vector<size_m>({4, 3}), "complex * real: dtype / shape");
    EXPECT((r + z).type == dtype::Complex64 && (z / z).type == dtype::Complex64 && (z - r).type == dtype::Complex64,
           "complex arithmetic dtype");
    EXPECT(r.astype(dtype::Complex64).type == dtype::Complex64, "real -> complex64 cast");
    EXPECT(throws_runtime([&] { matrix::max(z, z); }), "max of complex64 did not throw");
    EXPECT(throws_runtime([&] { matrix::min(z, r); }), "min of complex64 did not throw");
    EXPECT(throws_runtime([&] { matrix::equal(z, z); }), "equal of complex64 did not throw");
    EXPECT(throws_runtime([&] { z.sum(1); }), "sum of complex64 did not throw");
    EXPECT(throws_runtime([&] { z.argmax(0); }), "argmax of complex64 did not throw");
    EXPECT(throws_runtime([&] { z.dot(z.transpose({1, 0})); }), "dot of complex64 did not throw");
    EXPECT(throws_runtime([&] { z.astype(dtype::Float); }), "complex64 -> Float did not throw");
}

// (a * b - c) / (a + b) with a [64, 33] complex64, b [33] complex64 broadcast over rows and c a
// float32 [64, 1] column promoted to complex64, against complex128 host arithmetic on the same
// float32 inputs: each part within 16 u of the operands' magnitudes (mul, sub, add and div each
// round a few times); a swapped part or wrong sign is O(1) off.  Plus a transposed complex view
// made contiguous (a bit-exact move).
CASE(gpu_complex64_arithmetic) {
    using cf = std::complex<float>;
    using cd = std::complex<double>;
    const size_m R = 64, Cc = 33;
    auto ar = randn((size_t)R * Cc * 2, 70), br = randn((size_t)Cc * 2, 71), cv = randn(R, 72);
    std::vector<cf> av(R * Cc), bv(Cc);
    for (size_t i = 0; i < av.size(); i++) av[i] = cf(ar[2 * i], ar[2 * i + 1]);
    for (size_t i = 0; i < bv.size(); i++) bv[i] = cf(br[2 * i], br[2 * i + 1]);
    matrix a = matrix::from_host<cf>({R, Cc}, av);
    matrix b = matrix::from_host<cf>({Cc}, bv);
    matrix c = matrix::from_host<float>({R, 1}, cv);
    matrix y = (a * b - c) / (a + b);
    matrix t = a.transpose({1, 0}).astype(dtype::Complex64, true);
    std::vector<matrix> outs{y, t};
    matrix::eval(outs);
    EXPECT(y.type == dtype::Complex64, "result dtype");
    auto yg = y.to_host<cf>();
    auto tg = t.to_host<cf>();
    const double u = std::ldexp(1.0, -24);
    for (size_t r = 0; r < R; r++)
        for (size_t j = 0; j < Cc; j++) {
            const cd A(av[r * Cc + j]), B(bv[j]), C(cv[r], 0.0);
            const cd num = A * B - C, den = A + B;
            const cd want = num / den;
            const double scale = (std::abs(A) * std::abs(B) + std::abs(C) + 4 * std::abs(den) * std::abs(want)) /
                                 std::abs(den);
            const cd got(yg[r * Cc + j]);
            EXPECT(std::abs(got.real() - want.real()) <= 16 * u * scale &&
                       std::abs(got.imag() - want.imag()) <= 16 * u * scale,
                   "complex (a*b - c)/(a + b) at " + std::to_string(r) + "," + std::to_string(j));
            EXPECT(std::memcmp(&tg[j * R + r], &av[r * Cc + j], sizeof(cf)) == 0, "complex transpose copy");
        }
}

// An f16 dense layer's weight gradient: loss = (x . W).sum(), so dL/dW = x^T . 1 and the Dot's
// vjp forms g^T . x, whose g^T is read M-major (no copy); against float64 host sums of the same
// f16 inputs (each output a sum of 64 products; f16 result rounding).
CASE(gpu_f16_dot_vjp) {
    const size_m M = 64, K = 96, N = 128;
    auto xf = randn((size_t)M * K, 80), wf = randn((size_t)K * N, 81, 0.1f);
    std::vector<_Float16> xh(xf.size()), wh(wf.size());
    for (size_t i = 0; i < xf.size(); i++) xh[i] = (_Float16)xf[i];
    for (size_t i = 0; i < wf.size(); i++) wh[i] = (_Float16)wf[i];
    matrix x = matrix::from_host<_Float16>({M, K}, xh);
    matrix W = matrix::from_host<_Float16>({K, N}, wh);
    matrix y = x.dot(W);
    matrix t = matrix::from_host<_Float16>({M, N}, std::vector<_Float16>((size_t)M * N, (_Float16)0.25f));
    matrix loss = (y * t).sum();
    std::vector<matrix> outs{loss}, params{W, x};
    std::vector<matrix> grads = matrix::build_grad_graph(outs, params);
    matrix::eval(grads);
    auto gw = grads[0].to_host<_Float16>();
    auto gx = grads[1].to_host<_Float16>();
    double err = 0, mag = 0;
    for (size_t k = 0; k < K; k++)
        for (size_t n = 0; n < N; n++) {
            double ref = 0;                     // dL/dW[k, n] = sum_m x[m, k] * 0.25
            for (size_t m = 0; m < M; m++) ref += 0.25 * (double)(float)xh[m * K + k];
            err += ((double)(float)gw[k * N + n] - ref) * ((double)(float)gw[k * N + n] - ref);
            mag += ref * ref;
        }
    EXPECT(std::sqrt(err / mag) <= 2e-3, "f16 weight gradient (g^T . x) beyond 2e-3 normwise");
    err = mag = 0;
    for (size_t m = 0; m < M; m++)
        for (size_t k = 0; k < K; k++) {
            double ref = 0;                     // dL/dx[m, k] = sum_n 0.25 * W[k, n]
            for (size_t n = 0; n < N; n++) ref += 0.25 * (double)(float)wh[k * N + n];
            err += ((double)(float)gx[m * K + k] - ref) * ((double)(float)gx[m * K + k] - ref);
            mag += ref * ref;
        }
    EXPECT(std::sqrt(err / mag) <= 2e-3, "f16 input gradient (g . W^T) beyond 2e-3 normwise");
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    if (mode == "cpu") {
        run("shapes_broadcast_and_reduce", shapes_broadcast_and_reduce);
        run("shapes_dot_and_conv", shapes_dot_and_conv);
        run("views_share_storage", views_share_storage);
        run("grad_graph_structure", grad_graph_structure);
        run("complex_construction_rules", complex_construction_rules);
    } else {
        run("gpu_add_then_rowsum", gpu_add_then_rowsum);
        run("gpu_fused_reduction_lifecycle", gpu_fused_reduction_lifecycle);
        run("gpu_dense_bias_relu_lifecycle", gpu_dense_bias_relu_lifecycle);
        run("gpu_grouped_reductions", gpu_grouped_reductions);
        run("gpu_reductions_and_views", gpu_reductions_and_views);
        run("gpu_dot_batched_broadcast", gpu_dot_batched_broadcast);
        run("gpu_conv2d_nchw_views", gpu_conv2d_nchw_views);
        run("gpu_mlp_training_step_compile_once", gpu_mlp_training_step_compile_once);
        run("gpu_value_and_grad", gpu_value_and_grad);
        run("gpu_complex64_arithmetic", gpu_complex64_arithmetic);
        run("gpu_f16_dot_vjp", gpu_f16_dot_vjp);
    }
    return g_fail ? 1 : 0;
}
