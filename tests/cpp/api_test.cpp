// api_test.cpp -- the reference's graph API spellings and forward-mode autodiff.
//
// Written against the names matrix.h declares (compile_metal / execute_metal / eval_metal,
// at<T>(), the variadic matrix::eval, leaf_scalar / mark_changed, make_leaf / detach,
// jit_graph_gpu / grad_graph_gpu / multi_jit_graph_gpu, value_and_grad and grad on one matrix,
// Primitive::get_inputs / invalidate_pass / jvp), so a graph of the reference compiles unchanged.
//
//   api_test cpu   graph building only: get_inputs, invalidate_pass, at<T> on leaves, the shapes of
//                  build_jvp_graph's tangents; touches no device
//   api_test gpu   evaluated on the GPU against double-precision host loops: every spelling above,
//                  and the jvp of a 3-layer MLP against central finite differences in float64
//
// Prints "PASS <name>" / "FAIL <name>: <why>" per case; exit status 1 if any case failed.
#include "../../matrix_amd/host/matrix.hpp"

#include <cmath>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

static int g_fail = 0;

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

template <typename E, typename F>
static bool throws(F&& f) {
    try { f(); } catch (const E&) { return true; }
    return false;
}

static std::vector<float> randn(size_t n, uint64_t seed, float scale = 1.0f) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g) * scale;
    return v;
}

// ------------------------------------------------------------------ cpu
static void inputs_and_invalidation() {
    matrix a = matrix::from_host<float>({4, 3}, randn(12, 1));
    matrix b = matrix::leaf_scalar(2.0f);
    matrix c = matrix::from_host<float>({3}, randn(3, 2));
    matrix y = a * b;              // depends on a, b
    matrix z = (y + c).sum(1);     // depends on a, b, c
    matrix w = c * c;              // depends on c only
    std::vector<matrix> in = y.tape->get_inputs();
    EXPECT(in.size() == 2 && in[0].storage == a.storage && in[1].storage == b.storage, "get_inputs order");
    // pretend a whole execute happened, then change b on the host
    for (matrix* m : {&y, &z, &w}) m->tape->evaluated = true;
    z.tape->input_at(0).tape->evaluated = true;                 // y + c
    *static_cast<float*>(b.host_data()) = 3.0f;
    b.mark_changed();
    EXPECT(z.tape->invalidate_pass(1), "z depends on the changed leaf");
    EXPECT(!z.tape->evaluated && !y.tape->evaluated, "invalidated along the path");
    EXPECT(!w.tape->invalidate_pass(1) && w.tape->evaluated, "w does not depend on b");
    EXPECT(z.tape->invalidate_pass(1) && !z.tape->evaluated, "the same pass again is memoised");
    // after a new evaluation the version is current: nothing to invalidate in the next pass
    for (matrix* m : {&y, &z}) m->tape->evaluated = true;
    z.tape->input_at(0).tape->evaluated = true;
    EXPECT(!z.tape->invalidate_pass(2) && z.tape->evaluated, "no change since: stays evaluated");
}

static void at_on_leaves() {
    std::vector<int32_t> v(24);
    for (int i = 0; i < 24; i++) v[i] = i * 3;
    matrix m = matrix::from_host<int32_t>({2, 3, 4}, v);
    EXPECT(m.at<int32_t>(1, 2, 3) == 23 * 3, "at(1,2,3)");
    matrix t = m.transpose({2, 0, 1});                       // a view: strides honoured
    EXPECT(t.at<int32_t>(3, 1, 2) == 23 * 3, "at through a transposed view");
    EXPECT(throws<std::runtime_error>([&] { m.at<float>(0, 0, 0); }), "type mismatch");
    EXPECT(throws<std::runtime_error>([&] { m.at<int32_t>(0, 0); }), "rank mismatch");
    EXPECT(throws<std::out_of_range>([&] { m.at<int32_t>(0, 3, 0); }), "index out of range");
    m.at<int32_t>(0, 0, 0) = -7;                             // writes the leaf's host values
    EXPECT(m.to_host<int32_t>()[0] == -7, "write through at()");
    matrix s = matrix::leaf_scalar(1.5f);
    EXPECT(s.dims == 0 && s.at<float>() == 1.5f, "leaf_scalar");
    matrix h = matrix::scalar((_Float16)0.25f);
    EXPECT(h.type == dtype::Float16 && (float)h.at<_Float16>() == 0.25f, "at<_Float16>");
}

static void jvp_graph_shapes() {
    matrix x = matrix::leaf({5, 4}), w = matrix::leaf({4, 3}), b = matrix::leaf({3});
    matrix y = matrix::max(x.dot(w) + b, matrix::scalar(0.0f)).sum(1);
    std::vector<matrix> outs{y}, ins{w, b}, tans{matrix::leaf({4, 3}), matrix::leaf({3})};
    std::vector<matrix> ty = matrix::build_jvp_graph(outs, ins, tans);
    EXPECT(ty.size() == 1 && ty[0].shape_vec() == std::vector<size_m>{5}, "tangent of y has y's shape");
    std::vector<matrix> bad{matrix::leaf({4, 4}), matrix::leaf({3})};
    EXPECT(throws<std::invalid_argument>([&] { matrix::build_jvp_graph(outs, ins, bad); }), "tangent shape checked");
    // no dependence: zero tangent
    matrix c = x.sum(0);
    std::vector<matrix> o2{c};
    std::vector<matrix> tz = matrix::build_jvp_graph(o2, ins, tans);
    EXPECT(!tz[0].tape && tz[0].shape_vec() == std::vector<size_m>{4}, "independent output: zeros");
}

// ------------------------------------------------------------------ gpu
static void metal_spellings_and_at() {
    auto av = randn(64 * 32, 3), bv = randn(32, 4);
    matrix a = matrix::from_host<float>({64, 32}, av), b = matrix::from_host<float>({32}, bv);
    matrix c = a + b;
    matrix s = c.sum(1);
    c.compile_metal();
    c.execute_metal();
    for (int i = 0; i < 64; i += 7)
        for (int j = 0; j < 32; j += 5) EXPECT(c.at<float>(i, j) == av[i * 32 + j] + bv[j], "execute_metal + at");
    s.eval_metal();
    double r = 0;
    for (int j = 0; j < 32; j++) r += (double)av[5 * 32 + j] + bv[j];
    EXPECT(std::fabs(s.at<float>(5) - r) <= 1e-4 * 32, "eval_metal + at");
    // variadic eval: a matrix and a vector of them in one call
    matrix d = a * 2.0f, e = a - 1.0f;
    std::vector<matrix> rest{e};
    matrix::eval(d, rest);
    EXPECT(d.at<float>(3, 4) == av[3 * 32 + 4] * 2.0f && e.at<float>(3, 4) == av[3 * 32 + 4] - 1.0f, "eval(args...)");
    // at() caches the host copy per execute: a new execute after new inputs is seen
    matrix f = a * matrix::leaf_scalar(3.0f);
    matrix k = f.tape->input_at(1);
    f.eval();
    EXPECT(f.at<float>(0, 0) == av[0] * 3.0f, "before the change");
    *static_cast<float*>(k.host_data()) = 5.0f;
    k.mark_changed();
    f.clear_trace_checks();
    f.execute_metal();
    EXPECT(f.at<float>(0, 0) == av[0] * 5.0f, "at() after mark_changed + execute");
    // make_leaf / detach: the values stay, the graph goes
    matrix g = (a * a).sum(0);
    g.make_leaf();
    EXPECT(!g.tape && std::fabs(g.at<float>(2) - [&] {
        double t = 0;
        for (int i = 0; i < 64; i++) t += (double)av[i * 32 + 2] * av[i * 32 + 2];
        return t;
    }()) <= 1e-3, "make_leaf keeps the values");
    matrix h = g + 1.0f;                                       // a detached leaf feeds a new graph
    h.eval();
    EXPECT(h.at<float>(2) == g.at<float>(2) + 1.0f, "a made leaf as an input");
    matrix u = a + 1.0f, w = a + 2.0f;
    std::vector<matrix> uw{w};
    matrix::eval(u, uw);
    matrix::detach(u, uw);
    EXPECT(!u.tape && !uw[0].tape && u.at<float>(1, 1) == av[33] + 1.0f, "detach");
}

static void compiled_subgraphs() {
    auto wv = randn(16 * 8, 5, 0.25f);
    matrix W = matrix::from_host<float>({16, 8}, wv);
    auto f = matrix::jit_graph_gpu([&](matrix x) { return matrix::max(x.dot(W), matrix::scalar(0.0f)); },
                                   matrix::leaf({4, 16}));
    for (int call = 0; call < 3; call++) {
        auto xv = randn(4 * 16, 40 + call);
        matrix x = matrix::from_host<float>({4, 16}, xv);
        matrix y = f(x);
        y.eval();
        for (int i = 0; i < 4; i++)
            for (int j = 0; j < 8; j++) {
                double t = 0;
                for (int k = 0; k < 16; k++) t += (double)xv[i * 16 + k] * wv[k * 8 + j];
                EXPECT(std::fabs(y.at<float>(i, j) - std::max(t, 0.0)) <= 1e-5, "jit_graph_gpu call " + std::to_string(call));
            }
    }
    // an input that is itself a lazy node, in a strided layout: packed before the call
    auto zv = randn(16 * 4, 50);
    matrix zt = matrix::from_host<float>({16, 4}, zv).transpose({1, 0}) * 2.0f;   // [4, 16]
    matrix y2 = f(zt);
    y2.eval();
    double t = 0;
    for (int k = 0; k < 16; k++) t += 2.0 * zv[k * 4 + 1] * wv[k * 8 + 3];
    EXPECT(std::fabs(y2.at<float>(1, 3) - std::max(t, 0.0)) <= 1e-5, "jit on a lazy strided input");
    // grad_graph_gpu: d/dx sum(x * x * 3) = 6 x
    auto gf = matrix::grad_graph_gpu([](matrix x) { return (x * x * 3.0f).sum(); }, matrix::leaf({10}));
    auto xv = randn(10, 60);
    matrix gx = gf(matrix::from_host<float>({10}, xv));
    gx.eval();
    for (int i = 0; i < 10; i++) EXPECT(std::fabs(gx.at<float>(i) - 6.0 * xv[i]) <= 1e-5, "grad_graph_gpu");
    // multi_jit_graph_gpu: two outputs of one call, run once
    auto mf = matrix::multi_jit_graph_gpu(
        [](std::vector<matrix> p) { return std::vector<matrix>{p[0] + p[1], (p[0] * p[1]).sum(0)}; },
        {matrix::leaf({3, 5}), matrix::leaf({5})});
    auto pv = randn(15, 61), qv = randn(5, 62);
    std::vector<matrix> outs = mf({matrix::from_host<float>({3, 5}, pv), matrix::from_host<float>({5}, qv)});
    matrix::eval(outs);
    for (int j = 0; j < 5; j++) {
        double col = 0;
        for (int i = 0; i < 3; i++) {
            EXPECT(outs[0].at<float>(i, j) == pv[i * 5 + j] + qv[j], "multi_jit output 0");
            col += (double)pv[i * 5 + j] * qv[j];
        }
        EXPECT(std::fabs(outs[1].at<float>(j) - col) <= 1e-5, "multi_jit output 1");
    }
    // grad_graph_gpu over several inputs: d/dp sum(p * q) = q, d/dq = column sums of p
    auto gg = matrix::grad_graph_gpu([](std::vector<matrix> p) { return std::vector<matrix>{(p[0] * p[1]).sum()}; },
                                     std::vector<matrix>{matrix::leaf({3, 5}), matrix::leaf({5})});
    std::vector<matrix> grads = gg({matrix::from_host<float>({3, 5}, pv), matrix::from_host<float>({5}, qv)});
    matrix::eval(grads);
    for (int j = 0; j < 5; j++) {
        double col = 0;
        for (int i = 0; i < 3; i++) {
            EXPECT(grads[0].at<float>(i, j) == qv[j], "grad_graph_gpu (vector) d/dp");
            col += pv[i * 5 + j];
        }
        EXPECT(std::fabs(grads[1].at<float>(j) - col) <= 1e-5, "grad_graph_gpu (vector) d/dq");
    }
    // value_and_grad / grad on one matrix
    auto vg = matrix::value_and_grad([](matrix x) { return (x * x).sum(); });
    auto [val, g1] = vg(matrix::from_host<float>({10}, xv));
    double r = 0;
    for (float v : xv) r += (double)v * v;
    EXPECT(std::fabs(val.at<float>() - r) <= 1e-4 * r && std::fabs(g1.at<float>(4) - 2.0 * xv[4]) <= 1e-5,
           "value_and_grad(matrix)");
    matrix g2 = matrix::grad([](matrix x) { return (x * x).sum(); })(matrix::from_host<float>({10}, xv));
    EXPECT(std::fabs(g2.at<float>(7) - 2.0 * xv[7]) <= 1e-5, "grad(matrix)");
}

// y = sum((relu(relu(x W0 + b0) W1 + b1) W2 + b2 - t)^2) in float64 on the host
struct Mlp {
    size_m B, D[4];
};

static double host_loss(const Mlp& s, const std::vector<double>& x, const std::vector<std::vector<double>>& W,
                        const std::vector<std::vector<double>>& b, const std::vector<double>& t) {
    std::vector<double> h = x;
    for (int l = 0; l < 3; l++) {
        const size_m din = s.D[l], dout = s.D[l + 1];
        std::vector<double> z((size_t)s.B * dout);
        for (size_m i = 0; i < s.B; i++)
            for (size_m j = 0; j < dout; j++) {
                double acc = b[l][j];
                for (size_m k = 0; k < din; k++) acc += h[(size_t)i * din + k] * W[l][(size_t)k * dout + j];
                z[(size_t)i * dout + j] = l < 2 ? std::max(acc, 0.0) : acc;
            }
        h.swap(z);
    }
    double loss = 0;
    for (size_t i = 0; i < h.size(); i++) loss += (h[i] - t[i]) * (h[i] - t[i]);
    return loss;
}

static void mlp_jvp_against_finite_differences() {
    const Mlp s{16, {32, 48, 40, 6}};
    auto xv = randn((size_t)s.B * s.D[0], 70);
    auto tv = randn((size_t)s.B * s.D[3], 71);
    std::vector<matrix> params, tangents;
    std::vector<std::vector<double>> W(3), b(3), dW(3), db(3);
    for (int l = 0; l < 3; l++) {
        auto w = randn((size_t)s.D[l] * s.D[l + 1], 72 + l, 1.0f / std::sqrt((float)s.D[l]));
        auto bb = randn(s.D[l + 1], 75 + l, 0.1f);
        auto tw = randn(w.size(), 78 + l), tb = randn(bb.size(), 81 + l);
        params.push_back(matrix::from_host<float>({s.D[l], s.D[l + 1]}, w));
        params.push_back(matrix::from_host<float>({s.D[l + 1]}, bb));
        tangents.push_back(matrix::from_host<float>({s.D[l], s.D[l + 1]}, tw));
        tangents.push_back(matrix::from_host<float>({s.D[l + 1]}, tb));
        W[l].assign(w.begin(), w.end());
        b[l].assign(bb.begin(), bb.end());
        dW[l].assign(tw.begin(), tw.end());
        db[l].assign(tb.begin(), tb.end());
    }
    matrix x = matrix::from_host<float>({s.B, s.D[0]}, xv), t = matrix::from_host<float>({s.B, s.D[3]}, tv);
    matrix h = x;
    for (int l = 0; l < 3; l++) {
        matrix z = h.dot(params[2 * l]) + params[2 * l + 1];
        h = l < 2 ? matrix::max(z, matrix::scalar(0.0f)) : z;
    }
    matrix loss = ((h - t) * (h - t)).sum();
    std::vector<matrix> outs{loss};
    std::vector<matrix> jv = matrix::build_jvp_graph(outs, params, tangents);
    matrix::eval(jv);
    const double got = jv[0].at<float>();
    // central differences in float64 along the same tangent
    std::vector<double> xd(xv.begin(), xv.end()), td(tv.begin(), tv.end());
    const double eps = 1e-6;
    auto shifted = [&](double sgn) {
        std::vector<std::vector<double>> Wp = W, bp = b;
        for (int l = 0; l < 3; l++) {
            for (size_t i = 0; i < Wp[l].size(); i++) Wp[l][i] += sgn * eps * dW[l][i];
            for (size_t i = 0; i < bp[l].size(); i++) bp[l][i] += sgn * eps * db[l][i];
        }
        return host_loss(s, xd, Wp, bp, td);
    };
    const double fd = (shifted(1.0) - shifted(-1.0)) / (2 * eps);
    EXPECT(std::fabs(got - fd) <= 1e-4 * std::fabs(fd) + 1e-4,
           "jvp " + std::to_string(got) + " vs finite differences " + std::to_string(fd));
    // and the same directional derivative from the gradient: <grad, tangent>
    std::vector<matrix> grads = matrix::build_grad_graph(outs, params);
    matrix::eval(grads);
    double dot = 0;
    for (size_t p = 0; p < grads.size(); p++) {
        auto gv = grads[p].to_host<float>();
        auto tv2 = tangents[p].to_host<float>();
        for (size_t i = 0; i < gv.size(); i++) dot += (double)gv[i] * tv2[i];
    }
    EXPECT(std::fabs(dot - fd) <= 1e-4 * std::fabs(fd) + 1e-4, "<vjp, tangent> vs finite differences");
}

static void elementwise_jvps() {
    // jvp of each primitive against its closed form, tangent 1 on x
    auto xv = randn(64, 90), yv = randn(64, 91);
    for (float& v : yv) v = std::fabs(v) + 0.5f;
    matrix x = matrix::from_host<float>({8, 8}, xv), y = matrix::from_host<float>({8, 8}, yv);
    matrix one = matrix::ones({8, 8});
    std::vector<matrix> ins{x}, tans{one};
    auto dir = [&](matrix out) {
        std::vector<matrix> o{out};
        matrix j = matrix::build_jvp_graph(o, ins, tans)[0];
        j.eval();
        return j.to_host<float>();
    };
    auto d_div = dir(x / y), d_mul = dir(x * y), d_sub = dir(y - x);
    auto d_max = dir(matrix::max(x, y)), d_tr = dir(x.transpose({1, 0}) * 2.0f);
    auto d_sum = dir(x.sum(1)), d_mx = dir(x.max(1));
    for (int i = 0; i < 64; i++) {
        EXPECT(std::fabs(d_div[i] - 1.0 / yv[i]) <= 1e-6, "d(x/y)/dx");
        EXPECT(d_mul[i] == yv[i] && d_sub[i] == -1.0f, "d(x*y), d(y-x)");
        EXPECT(d_max[i] == (xv[i] > yv[i] ? 1.0f : 0.0f), "d max(x, y) (ties to y)");
        EXPECT(d_tr[i] == 2.0f, "d transpose");
    }
    for (int r = 0; r < 8; r++) {
        EXPECT(d_sum[r] == 8.0f, "d sum");
        EXPECT(d_mx[r] == 1.0f, "d max over an axis (one maximum)");
    }
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    if (mode == "cpu") {
        run("inputs_and_invalidation", inputs_and_invalidation);
        run("at_on_leaves", at_on_leaves);
        run("jvp_graph_shapes", jvp_graph_shapes);
    } else {
        run("metal_spellings_and_at", metal_spellings_and_at);
        run("compiled_subgraphs", compiled_subgraphs);
        run("elementwise_jvps", elementwise_jvps);
        run("mlp_jvp_against_finite_differences", mlp_jvp_against_finite_differences);
    }
    return g_fail ? 1 : 0;
}
