// matrix.cpp -- graph building, compile / execute, and reverse-mode autodiff for matrix.hpp.
//
// Node semantics follow the reference's Primitives (primitives.cpp): broadcast binary ops
// (Addition/Subtraction/Multiplication/DivisionPrimitive 397-1046, Max/MinPrimitive
// 2515-2824, equal Matrix.mm:14451-14540), one-axis reductions (Sum/Max/Min/ArgMax/ArgMin,
// primitives.cpp:1967-2972, 7584-7799), DotPrimitive (5464-5626), ConvolvePrimitive (192-396),
// AsType copies (Matrix.mm:8384-8413) and views.  Each node's compile() derives the collapsed
// descriptors its kernel consumes (collapse_dims*, Mods/Utils.mm:114-435) and allocates its
// output and workspace; execute() only launches.
#include "matrix.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <numeric>
#include <unordered_map>
#include <unordered_set>

#include "../../include/matrix_amd.h"
#include "../../include/matrix_amd_shape.h"

using matrix_amd::Storage;

namespace {

constexpr uint64_t kCap = (1ull << 31) - 1;    // collapse size cap (size_m indexing)

[[noreturn]] void fail_status(int st, const std::string& what) {
    throw std::runtime_error("matrix_amd: " + what + " failed (status " + std::to_string(st) + "): " + mx_last_error());
}
void check(int st, const std::string& what) {
    if (st != MX_OK) fail_status(st, what);
}

std::vector<size_m> contiguous_strides(const std::vector<size_m>& shape) {
    std::vector<size_m> st(shape.size());
    uint64_t acc = 1;
    for (int i = (int)shape.size() - 1; i >= 0; --i) {
        st[i] = (size_m)acc;
        acc *= shape[i];
    }
    return st;
}

uint64_t prod(const std::vector<size_m>& v) {
    uint64_t p = 1;
    for (auto x : v) p *= x;
    return p;
}

uint16_t host_f32_to_f16(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
uint16_t host_f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// One element of `type` holding `v` (static_cast semantics for the integer types).
void store_value(dtype type, double v, uint8_t* dst) {
    switch (type) {
    case dtype::Float: { float f = (float)v; std::memcpy(dst, &f, 4); break; }
    case dtype::Float16: { uint16_t h = host_f32_to_f16((float)v); std::memcpy(dst, &h, 2); break; }
    case dtype::BFloat16: { uint16_t h = host_f32_to_bf16((float)v); std::memcpy(dst, &h, 2); break; }
    case dtype::Int8: { int8_t x = (int8_t)(int64_t)v; std::memcpy(dst, &x, 1); break; }
    case dtype::UInt8: { uint8_t x = (uint8_t)(int64_t)v; std::memcpy(dst, &x, 1); break; }
    case dtype::Bool: { uint8_t x = v != 0.0; std::memcpy(dst, &x, 1); break; }
    case dtype::Int16: { int16_t x = (int16_t)(int64_t)v; std::memcpy(dst, &x, 2); break; }
    case dtype::UInt16: { uint16_t x = (uint16_t)(int64_t)v; std::memcpy(dst, &x, 2); break; }
    case dtype::Int32: { int32_t x = (int32_t)(int64_t)v; std::memcpy(dst, &x, 4); break; }
    case dtype::UInt32: { uint32_t x = (uint32_t)(int64_t)v; std::memcpy(dst, &x, 4); break; }
    case dtype::Int64: { int64_t x = (int64_t)v; std::memcpy(dst, &x, 8); break; }
    case dtype::UInt64: { uint64_t x = (uint64_t)v; std::memcpy(dst, &x, 8); break; }
    case dtype::Complex64: { const float c[2] = {(float)v, 0.0f}; std::memcpy(dst, c, 8); break; }
    default: throw std::invalid_argument("matrix: unsupported dtype");
    }
}

int norm_axis(int axis, uint32_t dims, const char* who) {
    if (axis < 0) axis += (int)dims;
    if (axis < 0 || axis >= (int)dims)
        throw std::invalid_argument(std::string("matrix::") + who + ": axis out of range for rank " + std::to_string(dims));
    return axis;
}

// A device buffer owned by a node (workspace).
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    ~DevBuf() { if (p) mx_hip_free(p); }
    void reserve(size_t b) {
        if (b <= bytes) return;
        if (p) { mx_hip_free(p); p = nullptr; }
        check(mx_hip_alloc(b, &p), "workspace allocation");
        bytes = b;
    }
};

char* dptr(const matrix& m) {
    if (!m.storage || !m.storage->dev) throw std::logic_error("matrix: operand has no device buffer (not compiled)");
    return static_cast<char*>(m.storage->dev) + m.offset * dtype_size(m.type);
}

}  // namespace

// ------------------------------------------------------------------ dtypes, storage, device
size_t dtype_size(dtype t) {
    switch (t) {
    case dtype::Float: case dtype::Int32: case dtype::UInt32: return 4;
    case dtype::Float16: case dtype::BFloat16: case dtype::Int16: case dtype::UInt16: return 2;
    case dtype::UInt8: case dtype::Int8: case dtype::Bool: return 1;
    case dtype::Int64: case dtype::UInt64: case dtype::Complex64: return 8;
    }
    return 0;
}

const char* dtype_name(dtype t) {
    static const char* names[] = {"Float", "Float16", "UInt8", "Int32", "Int16", "UInt32", "UInt16",
                                  "Bool", "Int8", "Complex64", "BFloat16", "Int64", "UInt64"};
    const unsigned i = (unsigned)t;
    return i < 13 ? names[i] : "?";
}

dtype promote_types(dtype a, dtype b) {
    if (a == b) return a;
    if (a == dtype::Complex64 || b == dtype::Complex64) return dtype::Complex64;
    if (a == dtype::Bool) return b;
    if (b == dtype::Bool) return a;
    if (is_floating(a) || is_floating(b)) return dtype::Float;     // Float, or a 16-bit float with another type
    const int wa = (int)dtype_size(a) * 8, wb = (int)dtype_size(b) * 8;
    if (is_unsigned(a) == is_unsigned(b)) return wa >= wb ? a : b;
    const dtype s = is_unsigned(a) ? b : a;                        // the signed one
    const int ws = is_unsigned(a) ? wb : wa, wu = is_unsigned(a) ? wa : wb;
    if (wu < ws) return s;
    if (wu == 64) return dtype::Float;
    return wu == 8 ? dtype::Int16 : dtype::Int32;
}

namespace matrix_amd {
namespace {
std::once_flag g_init_once;
int g_device = 0;
}  // namespace

void init(int device) {
    g_device = device;
    std::call_once(g_init_once, [] { check(mx_hip_init(g_device), "mx_hip_init"); });
}

Storage::~Storage() {
    if (dev && !borrowed) mx_hip_free(dev);
}

void Storage::allocate() {
    if (dev || bytes == 0) return;
    init(g_device);
    check(mx_hip_alloc(bytes, &dev), "device allocation");
}

void Storage::upload() {
    allocate();
    if (bytes) check(mx_hip_h2d(dev, host.data(), bytes, nullptr), "host-to-device copy");
    dev_stale = false;
}
}  // namespace matrix_amd

// ------------------------------------------------------------------ matrix basics
size_t matrix::total_size() const { return (size_t)prod(shp_); }

bool matrix::is_contiguous() const {
    uint64_t want = 1;
    for (int i = (int)dims - 1; i >= 0; --i) {
        if (shp_[i] != 1 && str_[i] != want) return false;
        want *= shp_[i];
    }
    return true;
}

matrix matrix::from_bytes(const std::vector<size_m>& shape, dtype type, const void* data) {
    matrix m;
    m.dims = (uint32_t)shape.size();
    m.type = type;
    m.shp_ = shape;
    m.str_ = contiguous_strides(shape);
    m.storage = std::make_shared<Storage>();
    m.storage->bytes = (size_t)prod(shape) * dtype_size(type);
    m.storage->host.assign(m.storage->bytes, 0);
    if (data && m.storage->bytes) std::memcpy(m.storage->host.data(), data, m.storage->bytes);
    m.storage->host_is_source = true;
    return m;
}

matrix matrix::leaf(const std::vector<size_m>& shape, dtype type) { return from_bytes(shape, type, nullptr); }

matrix matrix::full(const std::vector<size_m>& shape, double value, dtype type) {
    matrix m = from_bytes(shape, type, nullptr);
    const size_t es = dtype_size(type);
    uint8_t one[8];
    store_value(type, value, one);
    for (size_t i = 0; i < m.storage->bytes; i += es) std::memcpy(m.storage->host.data() + i, one, es);
    return m;
}


namespace {
uint64_t g_epoch = 1;     // versions of leaves changed on the host (mark_changed)

// A leaf whose values live on the device only (make_leaf / releaseTape of an evaluated node)
// gets them on the host, which becomes their source.
void take_to_host(Storage& st) {
    if (st.host_is_source) return;
    st.host.assign(st.bytes, 0);
    if (st.bytes && st.dev) check(mx_hip_d2h(st.host.data(), st.dev, st.bytes, nullptr), "device-to-host copy");
    st.host_is_source = true;
    st.dev_stale = false;
}
}  // namespace

void* matrix::host_data() {
    if (tape || !storage) throw std::logic_error("matrix::host_data: not a leaf");
    if (storage->borrowed) throw std::logic_error("matrix::host_data: a compiled graph's input placeholder");
    take_to_host(*storage);
    return storage->host.data();
}

void matrix::mark_changed() {
    if (tape || !storage) throw std::logic_error("matrix::mark_changed: not a leaf");
    take_to_host(*storage);
    storage->dev_stale = true;
    storage->leaf_version = ++g_epoch;
}

matrix matrix::leaf_scalar(float value, dtype type) { return scalar(value, type); }

void matrix::releaseTape() {
    if (!tape) return;
    if (!tape->evaluated) throw std::logic_error("matrix::releaseTape: the node is not evaluated");
    tape.reset();
    storage->host_is_source = false;    // the device holds the values
    storage->dev_stale = false;
}

void matrix::make_leaf() {
    if (tape && !tape->evaluated) eval();
    releaseTape();
}

void* matrix::host_view() {
    if (!storage) throw std::logic_error("matrix::at: empty matrix");
    if (storage->host_is_source) return storage->host.data();     // a leaf, or a view of one
    if (!tape) {
        take_to_host(*storage);
        return storage->host.data();
    }
    if (!tape->evaluated) eval();
    if (storage->host_version != storage->dev_version || storage->host.size() != storage->bytes) {
        storage->host.resize(storage->bytes);
        if (storage->bytes) check(mx_hip_d2h(storage->host.data(), storage->dev, storage->bytes, nullptr), "device-to-host copy");
        storage->host_version = storage->dev_version;
    }
    return storage->host.data();
}

bool Primitive::invalidate_pass(uint64_t current_pass_id) {
    if (last_visited_pass_id == current_pass_id) return !evaluated;
    last_visited_pass_id = current_pass_id;
    bool inv = false;
    uint64_t nv = version;
    for (uint32_t i = 0; i < num_inputs(); i++) {
        const matrix& in = input_at(i);
        if (in.tape) {
            if (in.tape->invalidate_pass(current_pass_id)) inv = true;
            if (in.tape->version > version) inv = true;
            nv = std::max(nv, in.tape->version);
        } else if (in.storage) {
            if (in.storage->leaf_version > version) inv = true;
            nv = std::max(nv, in.storage->leaf_version);
        }
    }
    if (inv) {
        evaluated = false;
        version = nv;
    }
    return inv;
}

void* matrix::device_ptr() const { return dptr(*this); }

matrix matrix::make_node(std::vector<size_m> shape, dtype type, std::shared_ptr<Primitive> prim) {
    matrix m;
    m.dims = (uint32_t)shape.size();
    m.type = type;
    m.str_ = contiguous_strides(shape);
    m.shp_ = std::move(shape);
    m.storage = std::make_shared<Storage>();
    m.storage->bytes = (size_t)prod(m.shp_) * dtype_size(type);
    m.tape = std::move(prim);
    return m;
}

matrix matrix::make_view(const matrix& base, std::vector<size_m> shape, std::vector<size_m> strides, size_t offset,
                         std::shared_ptr<Primitive> prim) {
    matrix m;
    m.dims = (uint32_t)shape.size();
    m.type = base.type;
    m.shp_ = std::move(shape);
    m.str_ = std::move(strides);
    m.offset = offset;
    m.storage = base.storage;
    m.tape = std::move(prim);
    return m;
}

// ------------------------------------------------------------------ primitives
namespace {

// A view: shares its input's storage, no kernel.  vjp maps the gradient back to the input.
struct ViewPrim : Primitive {
    enum Kind { Transpose, Reshape, Broadcast } kind;
    matrix in;
    std::vector<size_m> perm;          // Transpose: the axis order
    std::vector<size_m> out_shape;     // Reshape / Broadcast: the view's shape
    ViewPrim(Kind k, matrix x, std::vector<size_m> p = {}, std::vector<size_m> os = {})
        : kind(k), in(std::move(x)), perm(std::move(p)), out_shape(std::move(os)) {}
    const char* name() const override { return kind == Transpose ? "Transpose" : kind == Reshape ? "Reshape" : "Broadcast"; }
    uint32_t num_inputs() const override { return 1; }
    matrix& input_at(uint32_t) override { return in; }
    bool is_view() const override { return true; }
    void compile(const matrix&) override {}
    void execute(const matrix&) override {}
    std::vector<matrix> vjp(matrix& g) override {
        if (kind == Transpose) {
            std::vector<size_m> inv(perm.size());
            for (size_t i = 0; i < perm.size(); i++) inv[perm[i]] = (size_m)i;
            return {g.transpose(inv)};
        }
        if (kind == Reshape) return {g.reshape(in.shape_vec())};
        return {g.unbroadcast_shape(in.shape(), (int)in.dims)};
    }
    // primitives.cpp:3784 (transpose), :3451 (reshape), :3246 (broadcast)
    matrix jvp(std::vector<matrix>& t) override {
        if (kind == Transpose) return t[0].transpose(perm);
        if (kind == Reshape) return t[0].reshape(out_shape);
        return t[0].broadcast_to(out_shape);
    }
};

// Execute generation of the calling thread: run_schedule advances it once per execute.
thread_local uint64_t t_exec_gen = 0;

// A Dot node that also produces Max|Min(Add(Dot, bias), s): the dense layer's bias + ReLU.  The
// Max / Min node registers it at compile time (BinaryPrim::try_fuse_epilogue); the Dot's
// execute then launches mx_launch_batched_matmul_bias_act, which writes the Dot's, the Add's
// and the Max's outputs, and records the execute it did so in.  The Add and the Max skip their
// own launch only in that same execute.  The Add's and the Max's storage is held weakly (those
// nodes hold the Dot, not the other way round); bias and s are leaves.
struct DotEpilogue {
    matrix bias, s;
    std::weak_ptr<matrix_amd::Storage> z, h;
    std::weak_ptr<Primitive> add, actp;   // the Add and Max / Min nodes the Dot's launch stands in for
    int act = MX_OP_MAX;
    uint64_t gen = 0;
};

// A node scheduled by the execute now running on this thread (fused launches write a consumer's
// output only then: an evaluated consumer is a boundary other streams may be reading).
bool pending_now(const std::weak_ptr<Primitive>& w) {
    auto p = w.lock();
    return p && !p->evaluated && p->run_gen == t_exec_gen;
}

// MATRIX_AMD_FUSE_EPILOGUE=0 compiles Dot / Add / Max as three launches.
bool epilogue_fusion_on() {
    static const bool on = [] {
        const char* e = std::getenv("MATRIX_AMD_FUSE_EPILOGUE");
        return !e || std::atoi(e) != 0;
    }();
    return on;
}

// MATRIX_AMD_FUSE_MAXGRAD=0 keeps the four-node vjp of Max / Min.
bool maxgrad_fusion_on() {
    static const bool on = [] {
        const char* e = std::getenv("MATRIX_AMD_FUSE_MAXGRAD");
        return !e || std::atoi(e) != 0;
    }();
    return on;
}

// The gradient Max / Min send to one operand (side 0: a, side 1: b) as one node and one launch
// (mx_launch_max_grad) in place of the four nodes of their vjp, max|min(a, b), equal(b, that),
// 1 - mask and the product with g (primitives.cpp:2604-2608), with the same results bit for bit.
// g is contiguous with the broadcast's shape, as R is.
struct MaxGradPrim : Primitive {
    int op, side;
    matrix a, b, g;
    uint32_t cd = 0;
    uint32_t cs[MX_MAX_DIMS], sA[MX_MAX_DIMS], sB[MX_MAX_DIMS], sR[MX_MAX_DIMS];
    MaxGradPrim(int o, int sd, matrix x, matrix y, matrix gg)
        : op(o), side(sd), a(std::move(x)), b(std::move(y)), g(std::move(gg)) {}
    const char* name() const override { return op == MX_OP_MAX ? "MaxGrad" : "MinGrad"; }
    uint32_t num_inputs() const override { return 3; }
    matrix& input_at(uint32_t i) override { return i == 0 ? a : i == 1 ? b : g; }
    void compile(const matrix& out) override {
        uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
        check(mx_broadcast_shapes(a.shape(), a.strides(), a.dims, b.shape(), b.strides(), b.dims, os, ost, b1s, b1t, b2s,
                                  b2t), "broadcast");
        if (out.dims == 0) { cd = 0; return; }
        check(mx_collapse_dims3(os, b1t, b2t, ost, out.dims, kCap, cs, sA, sB, sR, &cd), "collapse_dims");
    }
    void execute(const matrix& out) override {
        check(mx_launch_max_grad(op, side, (int)a.type, (int)cd, cs, sR, sA, sB, dptr(out), dptr(a), dptr(b), dptr(g),
                                 stream), std::string("launch ") + name());
    }
    std::vector<matrix> vjp(matrix& gg) override {
        matrix mb = matrix::equal(b, op == MX_OP_MAX ? matrix::max(a, b) : matrix::min(a, b));
        matrix mask = side ? mb : 1.0f - mb;
        return {a.zeros(), b.zeros(), gg * mask};
    }
    // the mask is piecewise constant in a and b: only g's tangent passes
    matrix jvp(std::vector<matrix>& t) override {
        matrix mb = matrix::equal(b, op == MX_OP_MAX ? matrix::max(a, b) : matrix::min(a, b));
        return t[2] * (side ? mb : 1.0f - mb);
    }
};

// Broadcast binary op (and Equal): out = a op b with NumPy broadcasting.
// When a reduction over this node's last axis is compiled against it (ReducePrim::compile), the
// node also produces that reduction: execute() launches mx_launch_bcast_binary_reduce_rows, which
// writes this node's result and the reduction's output together, and counts the fused runs so the
// reduction knows when its output is already current.  The reduction's storage is held weakly
// (the reduction node holds this one, not the other way round).
struct BinaryPrim : Primitive {
    int op;
    matrix a, b;
    uint32_t cd = 0;
    uint32_t cs[MX_MAX_DIMS], sA[MX_MAX_DIMS], sB[MX_MAX_DIMS], sR[MX_MAX_DIMS];
    std::weak_ptr<matrix_amd::Storage> fused_out;   // the fused reduction's output
    std::weak_ptr<Primitive> fused_node;            // the fused reduction
    int fused_red_op = -1;
    uint32_t fused_n = 0;
    uint64_t fused_runs = 0;
    std::shared_ptr<DotEpilogue> epi_of;            // this Add / Max is part of a Dot's epilogue
    BinaryPrim(int o, matrix x, matrix y) : op(o), a(std::move(x)), b(std::move(y)) {}
    const char* name() const override {
        static const char* n[] = {"Add", "Sub", "Mul", "Divide", "Max", "Min", "Equal"};
        return n[op];
    }
    uint32_t num_inputs() const override { return 2; }
    matrix& input_at(uint32_t i) override { return i ? b : a; }
    void compile(const matrix& out) override {
        uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
        check(mx_broadcast_shapes(a.shape(), a.strides(), a.dims, b.shape(), b.strides(), b.dims, os, ost, b1s, b1t, b2s,
                                  b2t), "broadcast");
        if (out.dims == 0) { cd = 0; return; }
        check(mx_collapse_dims3(os, b1t, b2t, ost, out.dims, kCap, cs, sA, sB, sR, &cd), "collapse_dims");
        try_fuse_epilogue(out);
    }
    void try_fuse_epilogue(const matrix& out);
    // g can feed one MaxGradPrim per operand: one float dtype, g contiguous with the broadcast shape
    bool maxgrad_fusable(const matrix& g) const {
        const int ty = (int)a.type;
        if (!maxgrad_fusion_on() || (ty != MX_FLOAT32 && ty != MX_FLOAT16 && ty != MX_BFLOAT16)) return false;
        if (b.type != a.type || g.type != a.type || !g.storage || !g.is_contiguous() || g.offset != 0) return false;
        uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
        if (mx_broadcast_shapes(a.shape(), a.strides(), a.dims, b.shape(), b.strides(), b.dims, os, ost, b1s, b1t, b2s,
                                b2t) != MX_OK)
            return false;
        const uint32_t nd = std::max(a.dims, b.dims);
        return g.dims == nd && g.shape_vec() == std::vector<size_m>(os, os + nd);
    }
    void execute(const matrix& out) override {
        if (epi_of && epi_of->gen == t_exec_gen) return;   // the Dot's launch wrote this output just now
        if (auto red = fused_out.lock(); red && red->dev && fused_red_op >= 0 && pending_now(fused_node)) {
            check(mx_launch_bcast_binary_reduce_rows(op, fused_red_op, (int)a.type, (int)cd, cs, sR, sA, sB, fused_n,
                                                     dptr(out), dptr(a), dptr(b), red->dev, stream),
                  std::string("launch ") + name() + " + reduction");
            fused_runs++;
            return;
        }
        check(mx_launch_bcast_binary(op, (int)a.type, (int)cd, cs, sR, sA, sB, dptr(out), dptr(a), dptr(b), stream),
              std::string("launch ") + name());
    }
    std::vector<matrix> vjp(matrix& g) override {
        const size_m* as = a.shape();
        const size_m* bs = b.shape();
        switch (op) {
        case MX_OP_ADD: return {g.unbroadcast_shape(as, a.dims), g.unbroadcast_shape(bs, b.dims)};
        case MX_OP_SUB: return {g.unbroadcast_shape(as, a.dims), g.unbroadcast_shape(bs, b.dims) * -1.0f};
        case MX_OP_MUL: return {(g * b).unbroadcast_shape(as, a.dims), (g * a).unbroadcast_shape(bs, b.dims)};
        case MX_OP_DIV: {
            matrix ga = g / b;
            matrix gb = g * matrix::scalar(-1, a.type) * a / (b * b);
            return {ga.unbroadcast_shape(as, a.dims), gb.unbroadcast_shape(bs, b.dims)};
        }
        case MX_OP_MAX:
        case MX_OP_MIN: {
            if (maxgrad_fusable(g)) {
                auto side = [&](int sd) {
                    return matrix::make_node(g.shape_vec(), g.type, std::make_shared<MaxGradPrim>(op, sd, a, b, g));
                };
                return {side(0).unbroadcast_shape(as, a.dims), side(1).unbroadcast_shape(bs, b.dims)};
            }
            // ties send the gradient to b (primitives.cpp:2604-2608)
            matrix mask_b = matrix::equal(b, op == MX_OP_MAX ? matrix::max(a, b) : matrix::min(a, b));
            matrix mask_a = 1.0f - mask_b;
            return {(g * mask_a).unbroadcast_shape(as, a.dims), (g * mask_b).unbroadcast_shape(bs, b.dims)};
        }
        default: return {a.zeros(), b.zeros()};
        }
    }
    // primitives.cpp:496 (add), :653 (sub), :815 (mul), :975 (div), :2344 (equal), :2610 / :2765
    // (max / min: ties to b)
    matrix jvp(std::vector<matrix>& t) override {
        switch (op) {
        case MX_OP_ADD: return t[0] + t[1];
        case MX_OP_SUB: return t[0] - t[1];
        case MX_OP_MUL: return b * t[0] + a * t[1];
        case MX_OP_DIV: return (b * t[0] - a * t[1]) / (b * b);
        case MX_OP_MAX:
        case MX_OP_MIN: {
            matrix mask_b = matrix::equal(b, op == MX_OP_MAX ? matrix::max(a, b) : matrix::min(a, b));
            return t[0] * (1.0f - mask_b) + t[1] * mask_b;
        }
        default: {
            uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
            check(mx_broadcast_shapes(a.shape(), a.strides(), a.dims, b.shape(), b.strides(), b.dims, os, ost, b1s, b1t,
                                      b2s, b2t), "broadcast");
            return matrix::zeros(std::vector<size_m>(os, os + std::max(a.dims, b.dims)), a.type);
        }
        }
    }
};

// Where an axis max / min came from (primitives.cpp:1962-1965): 1/k at each of the k elements
// equal to the extremum (given with keepdims, so it broadcasts back along the axis), 0 elsewhere.
matrix extremum_weights(const matrix& input, const matrix& extremum, int axis) {
    matrix mask = matrix::equal(input, extremum);
    return mask / mask.sum(axis, true);
}

// One-axis reduction.
struct ReducePrim : Primitive {
    int op;
    matrix in;
    int axis;
    bool keepdims;
    uint32_t cd = 0, rstride = 0, n = 0;
    uint32_t cs[MX_MAX_DIMS], sOut[MX_MAX_DIMS], sIn[MX_MAX_DIMS];
    DevBuf ws;
    BinaryPrim* producer = nullptr;     // fused into this broadcast node (kept alive by `in`)
    uint64_t seen_runs = 0;
    ReducePrim(int o, matrix x, int ax, bool kd) : op(o), in(std::move(x)), axis(ax), keepdims(kd) {}
    const char* name() const override {
        static const char* nm[] = {"Sum", "Max", "Min", "ArgMax", "ArgMin"};
        return nm[op];
    }
    uint32_t num_inputs() const override { return 1; }
    matrix& input_at(uint32_t) override { return in; }
    void compile(const matrix& out) override {
        // the output is contiguous; keepdims does not change its layout
        std::vector<size_m> oshape;
        for (uint32_t i = 0; i < in.dims; i++)
            if ((int)i != axis) oshape.push_back(in.shape()[i]);
        const std::vector<size_m> ost = contiguous_strides(oshape);
        check(mx_collapse_dims_reduce2(in.shape(), ost.data(), in.strides(), in.dims, axis, 0, 1, kCap, cs, sOut, sIn,
                                       &cd), "collapse_dims_reduce");
        if (cd == 0) { cd = 1; cs[0] = 1; sOut[0] = 1; sIn[0] = 1; }
        rstride = in.strides()[axis];
        n = in.shape()[axis];
        size_t bytes = 0;
        check(mx_reduce_workspace_bytes(op, (int)in.type, rstride, n, (int)cd, cs, sOut, sIn, &bytes), "reduce workspace");
        if (bytes) ws.reserve(bytes);
        try_fuse(out);
    }
    // Fuse into the producing broadcast node when this reduces its last axis (rows of at most
    // 16 KiB, no split workspace) and the producer has no fused reduction yet.
    void try_fuse(const matrix& out) {
        auto* bp = dynamic_cast<BinaryPrim*>(in.tape.get());
        if (!bp || bp->fused_red_op >= 0 || bp->epi_of || in.dims == 0 || axis != (int)in.dims - 1 || ws.bytes || n == 0)
            return;
        if (!in.is_contiguous() || in.offset != 0 || (uint64_t)n * dtype_size(in.type) > 16384) return;
        bp->fused_out = out.storage;
        bp->fused_node = out.tape;
        bp->fused_red_op = op;
        bp->fused_n = n;
        producer = bp;
        seen_runs = bp->fused_runs;
    }
    void execute(const matrix& out) override {
        if (producer && producer->fused_runs != seen_runs) {   // the producer already wrote this output
            seen_runs = producer->fused_runs;
            return;
        }
        check(mx_launch_reduce(op, (int)in.type, rstride, n, (int)cd, cs, sOut, sIn, dptr(out), dptr(in), ws.p, ws.bytes,
                               stream), std::string("launch ") + name());
    }
    // Sum: primitives.cpp:2904-2910; Max / Min: the gradient split evenly between the elements
    // equal to the extremum (primitives.cpp:2044-2048, 2185-2189); ArgMax / ArgMin have none.
    std::vector<matrix> vjp(matrix& g) override {
        matrix gg = keepdims ? g : g.unsqueeze(axis);
        if (op == MX_RED_SUM) return {gg.broadcast_to(in.shape_vec())};
        if (op == MX_RED_MAX) return {extremum_weights(in, in.max(axis, true), axis) * gg};
        if (op == MX_RED_MIN) return {extremum_weights(in, in.min(axis, true), axis) * gg};
        throw std::logic_error(std::string("matrix: no vjp for ") + name());
    }
    // primitives.cpp:2912 (sum), :2051 / :2192 (max / min); an index has a zero tangent
    matrix jvp(std::vector<matrix>& t) override {
        if (op == MX_RED_SUM) return t[0].sum(axis, keepdims);
        if (op == MX_RED_MAX) return (extremum_weights(in, in.max(axis, true), axis) * t[0]).sum(axis, keepdims);
        if (op == MX_RED_MIN) return (extremum_weights(in, in.min(axis, true), axis) * t[0]).sum(axis, keepdims);
        std::vector<size_m> shape;
        for (uint32_t i = 0; i < in.dims; i++) {
            if ((int)i == axis) { if (keepdims) shape.push_back(1); }
            else shape.push_back(in.shape()[i]);
        }
        return matrix::zeros(shape, dtype::Int32);
    }
};

// C = A . Bt^T over the batch axes (a [..., M, K], bt [..., N, K]).
struct DotPrim : Primitive {
    matrix a, bt;
    uint32_t cd = 0, K = 0;
    uint32_t cs[MX_MAX_DIMS], sA[MX_MAX_DIMS], sB[MX_MAX_DIMS], sC[MX_MAX_DIMS];
    std::shared_ptr<DotEpilogue> epi;
    DevBuf ws;                      // split-K partials, reserved at compile
    DotPrim(matrix x, matrix y) : a(std::move(x)), bt(std::move(y)) {}
    const char* name() const override { return "Dot"; }
    uint32_t num_inputs() const override { return 2; }
    matrix& input_at(uint32_t i) override { return i ? bt : a; }
    void compile(const matrix& out) override {
        uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
        check(mx_broadcast_shapes_matmul(a.shape(), a.strides(), a.dims, bt.shape(), bt.strides(), bt.dims, os, ost, b1s,
                                         b1t, b2s, b2t), "broadcast_shapes_matmul");
        K = a.shape()[a.dims - 1];
        if (out.dims == 2) {
            cd = 2;
            for (int i = 0; i < 2; i++) { cs[i] = os[i]; sA[i] = b1t[i]; sB[i] = b2t[i]; sC[i] = ost[i]; }
        } else {
            check(mx_collapse_dims_matmul(os, b1t, b2t, ost, out.dims, kCap, cs, sA, sB, sC, &cd), "collapse_dims_matmul");
        }
        size_t bytes = 0;
        check(mx_matmul_workspace_bytes((int)a.type, (int)cd, cs, sA, sB, sC, K, &bytes), "matmul workspace");
        if (bytes) ws.reserve(bytes);
    }
    void execute(const matrix& out) override {
        if (epi) {
            auto z = epi->z.lock(), h = epi->h.lock();
            const auto& bs = epi->bias.storage;
            const auto& ss = epi->s.storage;
            if (z && h && z->dev && h->dev && bs->dev && !bs->dev_stale && ss->dev && !ss->dev_stale &&
                pending_now(epi->add) && pending_now(epi->actp)) {
                check(mx_launch_batched_matmul_bias_act((int)a.type, (int)cd, cs, sA, sB, sC, K, dptr(out), dptr(a),
                                                        dptr(bt), dptr(epi->bias), z->dev, epi->act, dptr(epi->s),
                                                        h->dev, ws.p, ws.bytes, stream),
                      "launch Dot + bias + activation");
                epi->gen = t_exec_gen;
                return;
            }
        }
        check(mx_launch_batched_matmul_ws((int)a.type, (int)cd, cs, sA, sB, sC, K, dptr(out), dptr(a), dptr(bt), ws.p,
                                          ws.bytes, stream),
              "launch Dot");
    }
    std::vector<matrix> vjp(matrix& g) override {
        // grad_a = g . Bt ; grad_Bt = g^T . A  (primitives.cpp:5550-5567)
        matrix ga = g.dot(bt, false);
        std::vector<size_m> axes(g.dims);
        std::iota(axes.begin(), axes.end(), 0);
        std::swap(axes[g.dims - 2], axes[g.dims - 1]);
        matrix gb = g.transpose(axes).dot(a, false);
        return {ga.unbroadcast_shape(a.shape(), a.dims), gb.unbroadcast_shape(bt.shape(), bt.dims)};
    }
    // primitives.cpp:5567: bilinear, with Bt already transposed
    matrix jvp(std::vector<matrix>& t) override { return t[0].dot(bt, true) + a.dot(t[1], true); }
};

// Max|Min(Add(Dot(...), bias), s) with bias and s leaves: the Dot launches all three (bias a row
// of N elements broadcast over the Dot's other axes, s one element, one float dtype throughout).
void BinaryPrim::try_fuse_epilogue(const matrix& out) {
    if ((op != MX_OP_MAX && op != MX_OP_MIN) || !epilogue_fusion_on()) return;
    const int ty = (int)out.type;
    if (ty != MX_FLOAT32 && ty != MX_FLOAT16 && ty != MX_BFLOAT16) return;
    if (b.tape || b.total_size() != 1 || b.type != out.type || fused_red_op >= 0) return;
    auto* add = dynamic_cast<BinaryPrim*>(a.tape.get());
    if (!add || add->op != MX_OP_ADD || add->epi_of || add->fused_red_op >= 0) return;
    auto* dot = dynamic_cast<DotPrim*>(add->a.tape.get());
    if (!dot || dot->epi) return;
    const matrix& t = add->a;
    const matrix& bias = add->b;
    if (t.type != out.type || bias.type != out.type || bias.tape || !bias.is_contiguous() || bias.offset != 0) return;
    if (t.dims < 2 || t.shape_vec() != a.shape_vec() || a.shape_vec() != out.shape_vec()) return;
    if (!t.is_contiguous() || t.offset != 0 || !a.is_contiguous() || a.offset != 0) return;
    const size_m N = t.shape()[t.dims - 1];
    if (bias.dims < 1 || bias.dims > t.dims || bias.shape()[bias.dims - 1] != N || bias.total_size() != N) return;
    auto e = std::make_shared<DotEpilogue>();
    e->bias = bias;
    e->s = b;
    e->z = a.storage;
    e->h = out.storage;
    e->add = a.tape;
    e->actp = out.tape;
    e->act = op;
    dot->epi = e;
    add->epi_of = e;
    epi_of = e;
}

// Strided copy with cast into a contiguous output.
struct CopyPrim : Primitive {
    matrix in;
    dtype to;
    uint32_t cd = 0;
    uint32_t cs[MX_MAX_DIMS], sD[MX_MAX_DIMS], sS[MX_MAX_DIMS];
    CopyPrim(matrix x, dtype t) : in(std::move(x)), to(t) {}
    const char* name() const override { return "AsType"; }
    uint32_t num_inputs() const override { return 1; }
    matrix& input_at(uint32_t) override { return in; }
    void compile(const matrix& out) override {
        if (in.dims == 0) { cd = 0; return; }
        const std::vector<size_m> dst = contiguous_strides(in.shape_vec());
        check(mx_collapse_dims2(in.shape(), dst.data(), in.strides(), in.dims, kCap, cs, sD, sS, &cd), "collapse_dims");
        (void)out;
    }
    void execute(const matrix& out) override {
        check(mx_launch_copy_strided((int)out.type, (int)in.type, (int)cd, cs, sD, sS, dptr(out), dptr(in), stream),
              "launch AsType");
    }
    std::vector<matrix> vjp(matrix& g) override { return {g.astype(in.type)}; }
    matrix jvp(std::vector<matrix>& t) override { return t[0].astype(to); }      // primitives.cpp:3588
};

// Channels-last convolution.
struct ConvPrim : Primitive {
    matrix in, k;
    std::vector<int> stride, pad_lo, pad_hi, dil, dil_lhs;
    int groups;
    bool flip;
    std::vector<uint32_t> ishape, kshape, oshape, ist, kst, ost;
    DevBuf ws;
    size_t ws_bytes = 0;
    ConvPrim(matrix x, matrix w, std::vector<int> s, std::vector<int> pl, std::vector<int> ph, std::vector<int> d,
             std::vector<int> dl, int g, bool f)
        : in(std::move(x)), k(std::move(w)), stride(std::move(s)), pad_lo(std::move(pl)), pad_hi(std::move(ph)),
          dil(std::move(d)), dil_lhs(std::move(dl)), groups(g), flip(f) {}
    const char* name() const override { return "Convolve"; }
    uint32_t num_inputs() const override { return 2; }
    matrix& input_at(uint32_t i) override { return i ? k : in; }
    void compile(const matrix& out) override {
        ishape = in.shape_vec(); kshape = k.shape_vec(); oshape = out.shape_vec();
        ist = in.strides_vec(); kst = k.strides_vec(); ost = out.strides_vec();
        check(mx_conv_workspace_bytes((int)in.type, (int)in.dims - 2, ishape.data(), kshape.data(), oshape.data(),
                                      ist.data(), kst.data(), ost.data(), groups, &ws_bytes), "conv workspace");
        if (ws_bytes) ws.reserve(ws_bytes);
    }
    void execute(const matrix& out) override {
        check(mx_launch_conv_nd((int)in.type, (int)in.dims - 2, ishape.data(), kshape.data(), oshape.data(), ist.data(),
                                kst.data(), ost.data(), pad_lo.data(), stride.data(), dil.data(), dil_lhs.data(), groups,
                                flip ? 1 : 0, dptr(out), dptr(in), dptr(k), ws.p, ws_bytes, stream),
              "launch Convolve");
    }
    std::vector<matrix> vjp(matrix&) override { throw std::logic_error("matrix: no vjp for Convolve"); }
    // primitives.cpp:298: bilinear, conv(dx, w) + conv(x, dw)
    matrix jvp(std::vector<matrix>& t) override {
        return matrix::conv(t[0], k, stride, pad_lo, pad_hi, dil, dil_lhs, groups, flip) +
               matrix::conv(in, t[1], stride, pad_lo, pad_hi, dil, dil_lhs, groups, flip);
    }
};

// The operands are cast to their promoted dtype first, as operator+ does (Matrix.mm:8312-8315).
// Ops the reference runs on real dtypes only (dispatch_type throws for Complex64, matrix.h:327-330,
// and no GPU kernel of theirs is instantiated for type 9).
void require_real(dtype t, const char* who) {
    if (is_complex(t)) throw std::runtime_error(std::string("matrix::") + who + ": Complex64 is not supported by this op");
}

matrix binary(int op, const matrix& x, const matrix& y) {
    if (!x.storage || !y.storage) throw std::invalid_argument("matrix: operand is empty");
    const dtype t = promote_types(x.type, y.type);
    if (op == MX_OP_MAX || op == MX_OP_MIN || op == MX_OP_EQ)
        require_real(t, op == MX_OP_MAX ? "max" : op == MX_OP_MIN ? "min" : "equal");
    matrix a = x.type == t ? x : x.astype(t);
    matrix b = y.type == t ? y : y.astype(t);
    uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
    if (mx_broadcast_shapes(a.shape(), a.strides(), a.dims, b.shape(), b.strides(), b.dims, os, ost, b1s, b1t, b2s,
                            b2t) != MX_OK)
        throw std::invalid_argument(std::string("matrix: ") + mx_last_error());
    const uint32_t nd = std::max(a.dims, b.dims);
    std::vector<size_m> shape(os, os + nd);
    return matrix::make_node(shape, t, std::make_shared<BinaryPrim>(op, a, b));
}

matrix reduce(int op, const matrix& x, int axis, bool keepdims, const char* who) {
    if (x.dims == 0) throw std::invalid_argument(std::string("matrix::") + who + ": rank-0 input");
    require_real(x.type, who);
    axis = norm_axis(axis, x.dims, who);
    std::vector<size_m> shape;
    for (uint32_t i = 0; i < x.dims; i++) {
        if ((int)i == axis) { if (keepdims) shape.push_back(1); }
        else shape.push_back(x.shape()[i]);
    }
    const dtype t = (op == MX_RED_ARGMAX || op == MX_RED_ARGMIN) ? dtype::Int32 : x.type;
    return matrix::make_node(shape, t, std::make_shared<ReducePrim>(op, x, axis, keepdims));
}

}  // namespace

// ------------------------------------------------------------------ views and casts
matrix matrix::transpose(const std::vector<size_m>& order) const {
    if (order.size() != dims) throw std::invalid_argument("matrix::transpose: order must name every axis");
    std::vector<size_m> s(dims), st(dims);
    std::vector<bool> seen(dims, false);
    for (uint32_t i = 0; i < dims; i++) {
        if (order[i] >= dims || seen[order[i]]) throw std::invalid_argument("matrix::transpose: bad axis order");
        seen[order[i]] = true;
        s[i] = shp_[order[i]];
        st[i] = str_[order[i]];
    }
    return make_view(*this, s, st, offset, std::make_shared<ViewPrim>(ViewPrim::Transpose, *this, order));
}

matrix matrix::reshape(const std::vector<size_m>& new_shape) const {
    if (prod(new_shape) != prod(shp_)) throw std::invalid_argument("matrix::reshape: element count changes");
    if (!is_contiguous()) return astype(type, true).reshape(new_shape);
    return make_view(*this, new_shape, contiguous_strides(new_shape), offset,
                     std::make_shared<ViewPrim>(ViewPrim::Reshape, *this, std::vector<size_m>{}, new_shape));
}

matrix matrix::flatten(int start, int end) const {
    if (dims == 0) return reshape({1});
    start = norm_axis(start, dims, "flatten");
    end = norm_axis(end, dims, "flatten");
    if (end < start) throw std::invalid_argument("matrix::flatten: end before start");
    std::vector<size_m> s;
    for (int i = 0; i < start; i++) s.push_back(shp_[i]);
    uint64_t m = 1;
    for (int i = start; i <= end; i++) m *= shp_[i];
    s.push_back((size_m)m);
    for (uint32_t i = end + 1; i < dims; i++) s.push_back(shp_[i]);
    return reshape(s);
}

matrix matrix::unsqueeze(int axis) const {
    if (axis < 0) axis += (int)dims + 1;
    if (axis < 0 || axis > (int)dims) throw std::invalid_argument("matrix::unsqueeze: axis out of range");
    std::vector<size_m> s = shp_, st = str_;
    const size_m stride = axis < (int)dims ? str_[axis] * shp_[axis] : 1;
    s.insert(s.begin() + axis, 1);
    st.insert(st.begin() + axis, stride);
    return make_view(*this, s, st, offset, std::make_shared<ViewPrim>(ViewPrim::Reshape, *this, std::vector<size_m>{}, s));
}

matrix matrix::broadcast_to(const std::vector<size_m>& shape) const {
    if (shape.size() < dims) throw std::invalid_argument("matrix::broadcast_to: target rank below source rank");
    const size_t lead = shape.size() - dims;
    std::vector<size_m> st(shape.size(), 0);
    for (uint32_t i = 0; i < dims; i++) {
        if (shp_[i] == shape[lead + i]) st[lead + i] = str_[i];
        else if (shp_[i] == 1) st[lead + i] = 0;
        else throw std::invalid_argument("MatrixH: Incompatible shapes for broadcasting");
    }
    return make_view(*this, shape, st, offset,
                     std::make_shared<ViewPrim>(ViewPrim::Broadcast, *this, std::vector<size_m>{}, shape));
}

// A real dtype casts to Complex64 as (float(v), 0) (complex.h:22); Complex64 has no cast to a real dtype.
matrix matrix::astype(dtype t, bool make_contig) const {
    if (t == type && (!make_contig || is_contiguous())) return *this;
    if (is_complex(type) && !is_complex(t)) throw std::runtime_error("matrix::astype: Complex64 has no cast to a real dtype");
    return make_node(shp_, t, std::make_shared<CopyPrim>(*this, t));
}

// ------------------------------------------------------------------ ops
matrix operator+(const matrix& a, const matrix& b) { return binary(MX_OP_ADD, a, b); }
matrix operator-(const matrix& a, const matrix& b) { return binary(MX_OP_SUB, a, b); }
matrix operator*(const matrix& a, const matrix& b) { return binary(MX_OP_MUL, a, b); }
matrix operator/(const matrix& a, const matrix& b) { return binary(MX_OP_DIV, a, b); }

// max / min give the promoted dtype (Matrix.mm:13363-13376).  The reference leaves operands of
// another dtype uncast, so its kernel then reads them in the result's dtype; here they are cast
// first, which gives the same values whenever the operands already share the result's dtype.
matrix matrix::max(const matrix& a, const matrix& b) { return binary(MX_OP_MAX, a, b); }
matrix matrix::min(const matrix& a, const matrix& b) { return binary(MX_OP_MIN, a, b); }
matrix matrix::equal(const matrix& a, const matrix& b) { return binary(MX_OP_EQ, a, b); }

matrix matrix::sum(int axis, bool keepdims) const { return reduce(MX_RED_SUM, *this, axis, keepdims, "sum"); }
matrix matrix::sum(int start, int end, bool keepdims) const { return flatten(start, end).sum(start, keepdims); }
matrix matrix::sum() const { return flatten(0, -1).sum(0); }
matrix matrix::max(int axis, bool keepdims) const { return reduce(MX_RED_MAX, *this, axis, keepdims, "max"); }
matrix matrix::min(int axis, bool keepdims) const { return reduce(MX_RED_MIN, *this, axis, keepdims, "min"); }
matrix matrix::argmax(int axis, bool keepdims) const { return reduce(MX_RED_ARGMAX, *this, axis, keepdims, "argmax"); }
matrix matrix::argmin(int axis, bool keepdims) const { return reduce(MX_RED_ARGMIN, *this, axis, keepdims, "argmin"); }
matrix matrix::SumNoRed(int axis) const { return sum(axis, true); }

// Sums the gradient of a broadcast operand back to its shape (Matrix.mm:5425-5443).
matrix matrix::unbroadcast_shape(const size_m* target_shape, int target_dims) const {
    matrix result = *this;
    const int rank_diff = (int)dims - target_dims;
    if (rank_diff > 0) result = result.sum(0, rank_diff - 1, false);
    for (int i = 0; i < target_dims; i++)
        if (target_shape[i] == 1 && result.shape()[i] != 1) result = result.SumNoRed(i);
    return result;
}

// A float Bt whose N axis is unit-stride with 16-byte K rows (B contiguous as [..., K, N], seen
// through the transpose): the GEMM reads B in that layout -- the tile kernel (fp32 as 4-column
// rows, 16-bit types through transposing LDS reads) or, for at most 16 rows of A, the streaming
// kernel's N-major form -- so no packed copy is made.
static bool n_major_ok(const matrix& bt) {
    if (!is_floating(bt.type) || bt.dims < 2) return false;
    const uint32_t ce = 16 / (uint32_t)dtype_size(bt.type);
    const size_m* st = bt.strides();
    const size_m* sh = bt.shape();
    if (st[bt.dims - 2] != 1 || st[bt.dims - 1] % ce || sh[bt.dims - 2] % ce || bt.offset % ce) return false;
    for (uint32_t d = 0; d + 2 < bt.dims; d++)
        if (sh[d] > 1 && st[d] % ce) return false;
    return true;
}

// A float A given M-major (a transposed view whose M axis is unit-stride, the vjp's g^T) that the
// tile kernel reads from an M-major slot: 16-byte K rows, M a whole number of 16-byte units.
static bool m_major_ok(const matrix& a) {
    if (!is_floating(a.type) || a.dims < 2) return false;
    const uint32_t ce = 16 / (uint32_t)dtype_size(a.type);
    const size_m* st = a.strides();
    const size_m* sh = a.shape();
    if (st[a.dims - 2] != 1 || st[a.dims - 1] % ce || sh[a.dims - 2] % ce || a.offset % ce) return false;
    for (uint32_t d = 0; d + 2 < a.dims; d++)
        if (sh[d] > 1 && st[d] % ce) return false;
    return true;
}

// dot packs B^T contiguous (and A when it is a strided view) before the product, as the
// reference does (Matrix.mm:7068-7092) -- except a float B that is already N-major and a float A
// that is M-major.
matrix matrix::dot(const matrix& b, bool transposeB) const {
    if (dims < 2 || b.dims < 2) throw std::invalid_argument("matrix::dot requires both matrices to be at least 2D");
    require_real(type, "dot");
    require_real(b.type, "dot");
    matrix bt = b;
    if (!transposeB) {
        std::vector<size_m> axes(b.dims);
        std::iota(axes.begin(), axes.end(), 0);
        std::swap(axes[b.dims - 2], axes[b.dims - 1]);
        bt = b.transpose(axes);
    }
    if (!bt.is_contiguous() && !(bt.type == type && n_major_ok(bt))) bt = bt.astype(bt.type, true);
    matrix a = is_contiguous() || m_major_ok(*this) ? *this : astype(type, true);
    if (bt.type != a.type) bt = bt.astype(a.type, true);
    uint32_t os[MX_MAX_DIMS], ost[MX_MAX_DIMS], b1s[MX_MAX_DIMS], b1t[MX_MAX_DIMS], b2s[MX_MAX_DIMS], b2t[MX_MAX_DIMS];
    if (mx_broadcast_shapes_matmul(a.shape(), a.strides(), a.dims, bt.shape(), bt.strides(), bt.dims, os, ost, b1s, b1t,
                                   b2s, b2t) != MX_OK)
        throw std::invalid_argument(std::string("matrix::dot: ") + mx_last_error());
    const uint32_t nd = std::max(a.dims, bt.dims);
    return make_node(std::vector<size_m>(os, os + nd), a.type, std::make_shared<DotPrim>(a, bt));
}

// conv (Matrix.mm:12267-12333): output extent (dilated_in + lo + hi - dilated_k) / stride + 1.
matrix matrix::conv(const matrix& input, const matrix& kernel, const std::vector<int>& stride,
                    const std::vector<int>& pad_lo, const std::vector<int>& pad_hi,
                    const std::vector<int>& kernel_dilation, const std::vector<int>& input_dilation, int groups,
                    bool flip) {
    if (input.dims < 3 || input.dims != kernel.dims)
        throw std::invalid_argument("matrix::conv: input and kernel must have the same rank >= 3");
    const int ns = (int)input.dims - 2;
    auto chk = [&](const std::vector<int>& v, const char* what) {
        if ((int)v.size() != ns) throw std::invalid_argument(std::string("matrix::conv: ") + what + " needs one entry per spatial axis");
    };
    chk(stride, "stride"); chk(pad_lo, "padding"); chk(pad_hi, "padding"); chk(kernel_dilation, "kernel dilation");
    chk(input_dilation, "input dilation");
    if (input.type != kernel.type) throw std::invalid_argument("matrix::conv: input and kernel dtypes differ");
    require_real(input.type, "conv");
    if (groups < 1 || input.shape()[ns + 1] % groups || kernel.shape()[0] % groups ||
        input.shape()[ns + 1] / groups != kernel.shape()[ns + 1])
        throw std::invalid_argument("matrix::conv: channels do not match the kernel and groups");
    std::vector<size_m> out = {input.shape()[0]};
    for (int d = 0; d < ns; d++) {
        if (stride[d] < 1 || kernel_dilation[d] < 1 || input_dilation[d] < 1)
            throw std::invalid_argument("matrix::conv: stride and dilations must be >= 1");
        const int64_t din = ((int64_t)input.shape()[d + 1] - 1) * input_dilation[d] + 1;
        const int64_t dk = ((int64_t)kernel.shape()[d + 1] - 1) * kernel_dilation[d] + 1;
        const int64_t span = din + pad_lo[d] + pad_hi[d] - dk;
        if (span < 0) throw std::invalid_argument("matrix::conv: kernel larger than the padded input");
        out.push_back((size_m)(span / stride[d] + 1));
    }
    out.push_back(kernel.shape()[0]);
    return make_node(out, input.type, std::make_shared<ConvPrim>(input, kernel, stride, pad_lo, pad_hi, kernel_dilation,
                                                                 input_dilation, groups, flip));
}

matrix matrix::conv2d(const matrix& input, const matrix& kernel, int stride_h, int stride_w, int pad_h, int pad_w,
                      int dilation_h, int dilation_w, int groups, int input_dilation_h, int input_dilation_w,
                      bool flip) {
    return conv(input, kernel, {stride_h, stride_w}, {pad_h, pad_w}, {pad_h, pad_w}, {dilation_h, dilation_w},
                {input_dilation_h, input_dilation_w}, groups, flip);
}

// ------------------------------------------------------------------ compile / execute
namespace {

void compile_node(const matrix& m, std::unordered_set<const Primitive*>& seen) {
    if (!m.storage) throw std::invalid_argument("matrix: empty handle in the graph");
    if (!m.tape) {                                  // leaf: device copy of the host values
        if (!m.storage->borrowed && (!m.storage->dev || m.storage->dev_stale)) m.storage->upload();
        return;
    }
    if (!seen.insert(m.tape.get()).second) return;
    for (uint32_t i = 0; i < m.tape->num_inputs(); i++) compile_node(m.tape->input_at(i), seen);
    if (!m.tape->compiled) {
        if (!m.tape->is_view()) m.storage->allocate();
        m.tape->compile(m);
        m.tape->compiled = true;
    }
}

// ------------------------------------------------------------------ the executor
// execute_gpu launches the graph's unevaluated nodes in topological order.
// * Horizontal fusion: pending reductions of one float dtype over one collapsed descriptor that
//   do not depend on each other run as one mx_launch_reduce_group launch (a unit; up to 8
//   members), so several of them stream through HBM in one launch instead of paying a launch's
//   ramp-up and tail each (MATRIX_AMD_GROUP=0 launches every node on its own).  A reduction fused
//   into its broadcast producer is never grouped.  Units run in a topological order of units.
// * Streams: the pending nodes split into independent parts (weakly connected components of their
//   data dependencies, a group's members joined into one part: leaves and nodes evaluated by an
//   earlier execute do not connect anything); each part runs on one stream, and the parts take
//   the executor's streams round-robin (two by default; MATRIX_AMD_STREAMS=1 gives the
//   reference's single in-order queue).  Independent work thus overlaps -- one kernel's tail with
//   another's start -- while a connected graph such as a training step stays on one stream and
//   needs no cross-stream waits.
// Every stream then joins the calling thread's stream, which execute waits on once, as
// execute_metal commits and waits (Matrix.mm:8452-8475).
// What an execute launches: the pending nodes in `order` (a group's members together), node i on
// the executor's stream stream_of[i].  Computed on the first execute of a set of outputs and
// replayed while it holds -- the same outputs, every scheduled node pending again, every boundary
// node still evaluated (execute + clear_trace_checks, as a compiled graph runs) -- so a repeated
// execute spends no host time on walking, grouping and ordering the graph.
struct Schedule {
    std::vector<const Primitive*> roots;
    std::vector<matrix> nodes, leaves;
    std::vector<const Primitive*> boundary;
    std::vector<int> order;                              // node indices, a group's members together
    std::vector<int> group_of, stream_of;
    std::vector<std::vector<int>> groups;
    std::vector<bool> used;
};

struct Executor {
    std::vector<void*> streams;     // [0] is the thread's stream
    std::vector<void*> events;
    int count = 0;
    bool group = true;
    // the schedules of the last few output sets, most recent first; they hold their graphs.  Like
    // the streams, never destroyed: a thread-exit destructor freeing device memory could run
    // after the HIP runtime has shut down.
    static constexpr size_t kSchedules = 4;
    std::vector<Schedule>& schedules = *new std::vector<Schedule>();
    Executor() {
        const char* env = std::getenv("MATRIX_AMD_STREAMS");
        count = env ? std::atoi(env) : 2;
        if (count < 1) count = 1;
        if (count > 8) count = 8;
        const char* genv = std::getenv("MATRIX_AMD_GROUP");
        group = !genv || std::atoi(genv) != 0;
    }
    // The streams and events live until the process ends: releasing them from a thread-exit
    // destructor could run after the HIP runtime has shut down.
    void* stream(int i) {
        if (streams.empty()) {
            void* s0 = nullptr;
            check(mx_hip_stream_for_thread(&s0), "executor stream");
            streams.push_back(s0);
        }
        while ((int)streams.size() <= i) {
            void* s = nullptr;
            check(mx_hip_stream_create(&s), "executor stream");
            streams.push_back(s);
        }
        return streams[i];
    }
    void* event(int i) {
        while ((int)events.size() <= i) {
            void* e = nullptr;
            check(mx_hip_event_create(&e), "executor event");
            events.push_back(e);
        }
        return events[i];
    }
};

Executor& executor() {
    thread_local Executor ex;
    return ex;
}

// The pending nodes reachable from the outputs (inputs first), the leaves reached (uploaded at
// run time when written on the host) and the evaluated nodes the walk stopped at (the schedule's
// boundary).
struct Walk {
    std::vector<matrix> nodes, leaves;
    std::vector<const Primitive*> boundary;
    std::unordered_map<const Primitive*, int> index;
};

void collect(const matrix& m, Walk& w) {
    if (!m.tape) {
        w.leaves.push_back(m);
        return;
    }
    if (w.index.count(m.tape.get())) return;
    if (m.tape->evaluated) {
        w.boundary.push_back(m.tape.get());
        return;
    }
    if (!m.tape->compiled) throw std::logic_error("matrix: execute before compile");
    for (uint32_t i = 0; i < m.tape->num_inputs(); i++) collect(m.tape->input_at(i), w);
    w.index[m.tape.get()] = (int)w.nodes.size();
    w.nodes.push_back(m);
}

int find_root(std::vector<int>& parent, int i) {
    while (parent[i] != i) i = parent[i] = parent[parent[i]];
    return i;
}

// A reduction node that may join a group launch, and its group key (dtype and descriptor).
ReducePrim* groupable(Primitive* p) {
    auto* r = dynamic_cast<ReducePrim*>(p);
    if (!r || r->producer) return nullptr;
    const int t = (int)r->in.type;
    return (t == MX_FLOAT32 || t == MX_FLOAT16 || t == MX_BFLOAT16) ? r : nullptr;
}

std::vector<uint32_t> group_key(const ReducePrim* r) {
    std::vector<uint32_t> k = {(uint32_t)r->in.type, r->rstride, r->n, r->cd};
    for (uint32_t i = 0; i < r->cd; i++) { k.push_back(r->cs[i]); k.push_back(r->sOut[i]); k.push_back(r->sIn[i]); }
    return k;
}

struct KeyHash {
    size_t operator()(const std::vector<uint32_t>& k) const {
        size_t h = 1469598103934665603ull;
        for (uint32_t v : k) h = (h ^ v) * 1099511628211ull;
        return h;
    }
};

void launch_group(const std::vector<int>& members, const std::vector<matrix>& nodes, void* stream) {
    int ops[MX_REDUCE_GROUP_MAX];
    void* outs[MX_REDUCE_GROUP_MAX];
    const void* ins[MX_REDUCE_GROUP_MAX];
    void* ws[MX_REDUCE_GROUP_MAX];
    size_t wsb[MX_REDUCE_GROUP_MAX];
    const int n = (int)members.size();
    auto* r0 = static_cast<ReducePrim*>(nodes[members[0]].tape.get());
    for (int k = 0; k < n; k++) {
        auto* r = static_cast<ReducePrim*>(nodes[members[k]].tape.get());
        ops[k] = r->op;
        outs[k] = dptr(nodes[members[k]]);
        ins[k] = dptr(r->in);
        ws[k] = r->ws.p;
        wsb[k] = r->ws.bytes;
    }
    check(mx_launch_reduce_group(n, ops, (int)r0->in.type, r0->rstride, r0->n, (int)r0->cd, r0->cs, r0->sOut, r0->sIn,
                                 outs, ins, ws, wsb, stream),
          "launch reduction group");
}

Schedule build_schedule(std::vector<matrix>& ms, Executor& ex) {
    Walk w;
    for (auto& m : ms) collect(m, w);
    Schedule sc;
    for (auto& m : ms) sc.roots.push_back(m.tape.get());
    std::vector<matrix>& nodes = w.nodes;
    std::unordered_map<const Primitive*, int>& index = w.index;
    const int N = (int)nodes.size();
    std::vector<std::vector<int>> deps(N);               // pending inputs of each node
    for (int i = 0; i < N; i++) {
        Primitive* p = nodes[i].tape.get();
        for (uint32_t j = 0; j < p->num_inputs(); j++) {
            const matrix& in = p->input_at(j);
            if (!in.tape) continue;
            auto it = index.find(in.tape.get());
            if (it != index.end()) deps[i].push_back(it->second);
        }
    }

    // groups: greedy in topological order; a node joins an open group of its key when none of the
    // group's members is among its (transitive) pending ancestors
    std::vector<int> group_of(N, -1);
    std::vector<std::vector<int>> groups;
    if (ex.group) {
        std::vector<int> eidx(N, -1);                    // index among groupable nodes
        int E = 0;
        for (int i = 0; i < N; i++)
            if (groupable(nodes[i].tape.get())) eidx[i] = E++;
        if (E > 1) {
            const int W = (E + 63) / 64;
            std::vector<uint64_t> anc((size_t)N * W, 0);     // groupable ancestors, bitsets
            for (int i = 0; i < N; i++)
                for (int j : deps[i]) {
                    for (int w = 0; w < W; w++) anc[(size_t)i * W + w] |= anc[(size_t)j * W + w];
                    if (eidx[j] >= 0) anc[(size_t)i * W + eidx[j] / 64] |= 1ull << (eidx[j] % 64);
                }
            std::unordered_map<std::vector<uint32_t>, std::vector<int>, KeyHash> open;   // key -> group ids
            for (int i = 0; i < N; i++) {
                if (eidx[i] < 0) continue;
                auto& cand = open[group_key(static_cast<ReducePrim*>(nodes[i].tape.get()))];
                int gid = -1;
                for (int g : cand) {
                    if ((int)groups[g].size() >= MX_REDUCE_GROUP_MAX) continue;
                    bool dep = false;
                    for (int m : groups[g])
                        if (anc[(size_t)i * W + eidx[m] / 64] >> (eidx[m] % 64) & 1) { dep = true; break; }
                    if (!dep) { gid = g; break; }
                }
                if (gid < 0) {
                    gid = (int)groups.size();
                    groups.emplace_back();
                    cand.push_back(gid);
                }
                groups[gid].push_back(i);
                group_of[i] = gid;
            }
            for (size_t g = 0; g < groups.size(); g++)       // a group of one is a plain node
                if (groups[g].size() == 1) { group_of[groups[g][0]] = -1; groups[g].clear(); }
        }
    }

    // units: a group, or a node outside every group; run in a topological order of units (Kahn,
    // earliest first member first).  Should grouping ever close a cycle between two groups, every
    // node runs on its own in the original order.
    std::vector<int> order;                              // node indices, a group's members together
    {
        const int G = (int)groups.size();
        auto unit_of = [&](int i) { return group_of[i] >= 0 ? group_of[i] : G + i; };
        const int U = G + N;
        std::vector<int> indeg(U, 0), first(U, N);
        std::vector<std::vector<int>> succ(U);
        std::vector<bool> live(U, false);
        for (int i = 0; i < N; i++) {
            const int u = unit_of(i);
            live[u] = true;
            first[u] = std::min(first[u], i);
            for (int j : deps[i]) {
                const int v = unit_of(j);
                if (v != u) { succ[v].push_back(u); indeg[u]++; }
            }
        }
        std::vector<std::pair<int, int>> heap;           // (first member, unit), min-heap
        auto cmp = [](const std::pair<int, int>& a, const std::pair<int, int>& b) { return a > b; };
        for (int u = 0; u < U; u++)
            if (live[u] && indeg[u] == 0) heap.push_back({first[u], u});
        std::make_heap(heap.begin(), heap.end(), cmp);
        while (!heap.empty()) {
            std::pop_heap(heap.begin(), heap.end(), cmp);
            const int u = heap.back().second;
            heap.pop_back();
            if (u < G) for (int m : groups[u]) order.push_back(m);
            else order.push_back(u - G);
            for (int v : succ[u])
                if (--indeg[v] == 0) { heap.push_back({first[v], v}); std::push_heap(heap.begin(), heap.end(), cmp); }
        }
        if ((int)order.size() != N) {
            order.resize(N);
            std::iota(order.begin(), order.end(), 0);
            std::fill(group_of.begin(), group_of.end(), -1);
            groups.clear();
        }
    }

    // parts: union with every pending input, and a group's members with each other
    std::vector<int> parent(N);
    std::iota(parent.begin(), parent.end(), 0);
    auto unite = [&](int a, int b) {
        a = find_root(parent, a);
        b = find_root(parent, b);
        if (a != b) parent[std::max(a, b)] = std::min(a, b);
    };
    for (int i = 0; i < N; i++)
        for (int j : deps[i]) unite(i, j);
    for (auto& g : groups)
        for (size_t k = 1; k < g.size(); k++) unite(g[0], g[k]);

    const int K = ex.count;
    std::unordered_map<int, int> part_stream;
    sc.used.assign(K, false);
    sc.used[0] = true;
    sc.stream_of.assign(N, 0);
    for (int i : order) {
        if (nodes[i].tape->is_view()) continue;
        const int root = find_root(parent, i);
        auto it = part_stream.find(root);
        const int k = it != part_stream.end() ? it->second : (int)(part_stream.size() % K);
        if (it == part_stream.end()) part_stream.emplace(root, k);
        sc.used[k] = true;
        sc.stream_of[i] = k;
    }
    sc.order = std::move(order);
    sc.group_of = std::move(group_of);
    sc.groups = std::move(groups);
    sc.nodes = std::move(w.nodes);
    sc.leaves = std::move(w.leaves);
    sc.boundary = std::move(w.boundary);
    return sc;
}

bool schedule_holds(const Schedule& sc, const std::vector<matrix>& ms) {
    if (sc.roots.size() != ms.size()) return false;
    for (size_t i = 0; i < ms.size(); i++)
        if (sc.roots[i] != ms[i].tape.get()) return false;
    for (const matrix& n : sc.nodes)
        if (n.tape->evaluated) return false;
    for (const Primitive* b : sc.boundary)
        if (!b->evaluated) return false;
    return true;
}

void run_schedule(const Schedule& sc, Executor& ex) {
    t_exec_gen++;
    for (const matrix& l : sc.leaves)
        if (l.storage->dev_stale) l.storage->upload();      // leaf written on the host
    const auto& nodes = sc.nodes;
    for (const matrix& n : nodes) n.tape->run_gen = t_exec_gen;
    for (size_t oi = 0; oi < sc.order.size(); oi++) {
        const int i = sc.order[oi];
        Primitive* p = nodes[i].tape.get();
        if (!p->is_view()) {
            p->stream = ex.stream(sc.stream_of[i]);
            if (sc.group_of[i] >= 0) {                   // the whole group, then skip its members
                const auto& g = sc.groups[sc.group_of[i]];
                launch_group(g, nodes, p->stream);
                for (int m : g) {
                    nodes[m].tape->evaluated = true;
                    nodes[m].storage->dev_version++;
                }
                oi += g.size() - 1;
                continue;
            }
            p->execute(nodes[i]);
        }
        p->evaluated = true;
        nodes[i].storage->dev_version++;
    }
    void* s0 = ex.stream(0);
    int nev = 0;
    for (int k = 1; k < (int)sc.used.size(); k++) {      // join into the thread's stream
        if (!sc.used[k]) continue;
        void* e = ex.event(nev++);
        check(mx_hip_event_record(e, ex.stream(k)), "event record");
        check(mx_hip_stream_wait_event(s0, e), "stream wait");
    }
    check(mx_hip_sync(s0), "execute");
}

void run_graph(std::vector<matrix>& ms) {
    Executor& ex = executor();
    for (size_t c = 0; c < ex.schedules.size(); c++)
        if (schedule_holds(ex.schedules[c], ms)) {
            if (c) std::swap(ex.schedules[c], ex.schedules[0]);      // most recent first
            run_schedule(ex.schedules[0], ex);
            return;
        }
    Schedule sc = build_schedule(ms, ex);
    run_schedule(sc, ex);
    ex.schedules.insert(ex.schedules.begin(), std::move(sc));
    if (ex.schedules.size() > Executor::kSchedules) ex.schedules.pop_back();
}

void clear_node(const matrix& m, std::unordered_set<const Primitive*>& seen) {
    if (!m.tape || !seen.insert(m.tape.get()).second) return;
    m.tape->evaluated = false;
    for (uint32_t i = 0; i < m.tape->num_inputs(); i++) clear_node(m.tape->input_at(i), seen);
}

}  // namespace

void matrix::compile_gpu(std::vector<matrix>& ms) {
    matrix_amd::init();
    std::unordered_set<const Primitive*> seen;
    for (auto& m : ms) compile_node(m, seen);
}
void matrix::execute_gpu(std::vector<matrix>& ms) { run_graph(ms); }
void matrix::clear_trace_checks(std::vector<matrix>& ms) {
    std::unordered_set<const Primitive*> seen;
    for (auto& m : ms) clear_node(m, seen);
}
void matrix::eval(std::vector<matrix>& ms) {
    compile_gpu(ms);
    execute_gpu(ms);
}
void matrix::compile_gpu() { std::vector<matrix> v{*this}; compile_gpu(v); }
void matrix::execute_gpu() { std::vector<matrix> v{*this}; execute_gpu(v); }
void matrix::clear_trace_checks() { std::vector<matrix> v{*this}; clear_trace_checks(v); }
void matrix::eval() { std::vector<matrix> v{*this}; eval(v); }

std::vector<uint8_t> matrix::to_host_bytes() const {
    const size_t es = dtype_size(type);
    std::vector<uint8_t> full;
    if (storage->host_is_source) {                      // a leaf's host values, or a view of them
        full = storage->host;
    } else if (tape) {
        if (!tape->evaluated) { matrix self = *this; self.eval(); }
        full.resize(storage->bytes);
        if (storage->bytes) check(mx_hip_d2h(full.data(), storage->dev, storage->bytes, nullptr), "device-to-host copy");
    } else {                                            // a leaf whose values are on the device
        full.resize(storage->bytes);
        if (storage->bytes) check(mx_hip_d2h(full.data(), storage->dev, storage->bytes, nullptr), "device-to-host copy");
    }
    const size_t n = total_size();
    std::vector<uint8_t> out(n * es);
    std::vector<size_m> idx(dims, 0);
    for (size_t i = 0; i < n; i++) {
        uint64_t off = offset;
        for (uint32_t d = 0; d < dims; d++) off += (uint64_t)idx[d] * str_[d];
        std::memcpy(out.data() + i * es, full.data() + off * es, es);
        for (int d = (int)dims - 1; d >= 0; --d) {
            if (++idx[d] < shp_[d]) break;
            idx[d] = 0;
        }
    }
    return out;
}

// ------------------------------------------------------------------ autodiff (Matrix.mm:1327-1411)
namespace {
const void* node_id(const matrix& m) { return m.tape ? (const void*)m.tape.get() : (const void*)m.storage.get(); }
}  // namespace

std::vector<matrix> matrix::build_grad_graph(std::vector<matrix>& output_nodes, std::vector<matrix>& sample_input_nodes) {
    std::vector<const matrix*> topo;
    std::unordered_map<const void*, bool> depends;
    std::unordered_map<const void*, matrix> grads;
    std::unordered_set<const void*> params;
    for (auto& p : sample_input_nodes) params.insert(node_id(p));

    std::function<void(const matrix&)> dfs = [&](const matrix& m) {
        const void* id = node_id(m);
        if (depends.count(id)) return;
        bool dep = false;
        if (m.tape) {
            for (uint32_t i = 0; i < m.tape->num_inputs(); i++) {
                const matrix& in = m.tape->input_at(i);
                dfs(in);
                if (depends[node_id(in)]) dep = true;
            }
        }
        depends[id] = params.count(id) || dep;
        topo.push_back(&m);
    };
    for (auto& out : output_nodes) {
        dfs(out);
        if (depends[node_id(out)]) grads.insert({node_id(out), out.ones()});
    }
    for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
        const matrix& m = **it;
        if (!m.tape || !depends[node_id(m)]) continue;
        auto g = grads.find(node_id(m));
        if (g == grads.end()) continue;
        matrix current = g->second;
        std::vector<matrix> in_grads = m.tape->vjp(current);
        const uint32_t n = m.tape->num_inputs();
        if (in_grads.size() != n)
            throw std::logic_error("matrix: build_grad_graph => a vjp returned " + std::to_string(in_grads.size()) +
                                   " gradients for " + std::to_string(n) + " inputs");
        for (uint32_t i = 0; i < n; i++) {
            const void* in_id = node_id(m.tape->input_at(i));
            if (!depends[in_id]) continue;
            auto f = grads.find(in_id);
            if (f != grads.end()) f->second = f->second + in_grads[i];
            else grads.insert({in_id, in_grads[i]});
        }
    }
    std::vector<matrix> out;
    for (auto& p : sample_input_nodes) {
        auto f = grads.find(node_id(p));
        out.push_back(f != grads.end() ? f->second : p.zeros());
    }
    return out;
}

matrix matrix::build_grad_graph(matrix& output_node, matrix& sample_input_node) {
    std::vector<matrix> o{output_node}, p{sample_input_node};
    return build_grad_graph(o, p)[0];
}

std::function<std::pair<matrix, std::vector<matrix>>(const std::vector<matrix>&)> matrix::value_and_grad(
    std::function<matrix(std::vector<matrix>)> fn) {
    return [fn](const std::vector<matrix>& params) {
        std::vector<matrix> ps = params;
        matrix value = fn(ps);
        if (value.total_size() != 1)     // like MLX: a gradient needs a single-element output
            throw std::invalid_argument("matrix::value_and_grad: the function must return a single element");
        std::vector<matrix> outs{value};
        std::vector<matrix> grads = build_grad_graph(outs, ps);
        std::vector<matrix> all = grads;
        all.push_back(value);
        eval(all);
        return std::make_pair(value, grads);
    };
}

std::function<std::vector<matrix>(const std::vector<matrix>&)> matrix::grad(std::function<matrix(std::vector<matrix>)> fn) {
    auto vg = value_and_grad(std::move(fn));
    return [vg](const std::vector<matrix>& params) { return vg(params).second; };
}

std::function<std::pair<matrix, matrix>(const matrix&)> matrix::value_and_grad(std::function<matrix(matrix)> fn) {
    auto vg = value_and_grad(std::function<matrix(std::vector<matrix>)>([fn](std::vector<matrix> p) { return fn(p[0]); }));
    return [vg](const matrix& x) {
        auto r = vg({x});
        return std::make_pair(r.first, r.second[0]);
    };
}

std::function<matrix(const matrix&)> matrix::grad(std::function<matrix(matrix)> fn) {
    auto vg = value_and_grad(std::move(fn));
    return [vg](const matrix& x) { return vg(x).second; };
}

// ------------------------------------------------------------------ forward mode
std::vector<matrix> matrix::build_jvp_graph(std::vector<matrix>& output_nodes, std::vector<matrix>& input_nodes,
                                            std::vector<matrix>& input_tangents) {
    if (input_nodes.size() != input_tangents.size())
        throw std::invalid_argument("matrix::build_jvp_graph: one tangent per input");
    std::unordered_map<const void*, matrix> tan;
    for (size_t i = 0; i < input_nodes.size(); i++) {
        if (input_tangents[i].shape_vec() != input_nodes[i].shape_vec())
            throw std::invalid_argument("matrix::build_jvp_graph: a tangent's shape differs from its input's");
        tan.insert({node_id(input_nodes[i]), input_tangents[i]});
    }
    // the nodes that depend on an input, in topological order
    std::unordered_map<const void*, bool> depends;
    std::vector<const matrix*> topo;
    std::function<void(const matrix&)> dfs = [&](const matrix& m) {
        const void* id = node_id(m);
        if (depends.count(id)) return;
        bool dep = tan.count(id) > 0;
        if (m.tape && !dep)
            for (uint32_t i = 0; i < m.tape->num_inputs(); i++) {
                const matrix& in = m.tape->input_at(i);
                dfs(in);
                if (depends[node_id(in)]) dep = true;
            }
        depends[id] = dep;
        if (dep && !tan.count(id)) topo.push_back(&m);
    };
    for (auto& o : output_nodes) dfs(o);
    for (const matrix* m : topo) {
        std::vector<matrix> ts;
        for (uint32_t i = 0; i < m->tape->num_inputs(); i++) {
            const matrix& in = m->tape->input_at(i);
            auto it = tan.find(node_id(in));
            ts.push_back(it != tan.end() ? it->second : in.zeros());
        }
        tan.insert({node_id(*m), m->tape->jvp(ts)});
    }
    std::vector<matrix> out;
    for (auto& o : output_nodes) {
        auto it = tan.find(node_id(o));
        out.push_back(it != tan.end() ? it->second : o.zeros());
    }
    return out;
}

// ------------------------------------------------------------------ compiled sub-graphs
namespace {

// A graph traced once on placeholder leaves and compiled; each CompiledNodePrim runs it on its
// own inputs.  The placeholders borrow the inputs' device buffers for the run (no copy), and the
// nodes of every call share the graph's output buffers (MultiInputCompilePrimitive /
// CompiledNodePrimitive, primitives.cpp:3844-4200).
struct CompiledGraph {
    std::vector<matrix> samples, outputs;
    std::vector<matrix> order;              // the graph's nodes, inputs first
    std::vector<matrix> leaves;             // its other leaves (uploaded again when written)
};

std::shared_ptr<CompiledGraph> compile_subgraph(const std::vector<matrix>& sample_inputs,
                                                const std::function<std::vector<matrix>(std::vector<matrix>)>& build) {
    auto g = std::make_shared<CompiledGraph>();
    for (const matrix& s : sample_inputs) {
        if (!s.storage) throw std::invalid_argument("matrix::jit_graph_gpu: empty sample");
        matrix ph = matrix::leaf(s.shape_vec(), s.type);
        ph.storage->host.clear();
        ph.storage->host.shrink_to_fit();
        ph.storage->host_is_source = false;
        ph.storage->borrowed = true;
        ph.storage->dev_stale = false;
        g->samples.push_back(ph);
    }
    g->outputs = build(g->samples);
    for (const matrix& o : g->outputs)
        if (!o.tape) throw std::invalid_argument("matrix::jit_graph_gpu: an output is a leaf, not a computed node");
    matrix::compile_gpu(g->outputs);
    Walk w;
    for (auto& o : g->outputs) collect(o, w);
    g->order = std::move(w.nodes);
    for (auto& l : w.leaves)
        if (!l.storage->borrowed) g->leaves.push_back(l);
    return g;
}

struct CompiledNodePrim : Primitive {
    std::shared_ptr<CompiledGraph> graph;
    std::vector<matrix> ins;
    CompiledNodePrim(std::shared_ptr<CompiledGraph> g, std::vector<matrix> x) : graph(std::move(g)), ins(std::move(x)) {}
    const char* name() const override { return "CompiledGraph"; }
    uint32_t num_inputs() const override { return (uint32_t)ins.size(); }
    matrix& input_at(uint32_t i) override { return ins[i]; }
    void compile(const matrix&) override {}
    // One call's outputs are views sharing this node, so an execute runs it once for all of them.
    // Calls of one compiled graph share its output buffers: the last call run wins (as in the
    // reference).
    void execute(const matrix&) override {
        CompiledGraph& g = *graph;
        for (size_t i = 0; i < ins.size(); i++) g.samples[i].storage->dev = dptr(ins[i]);
        for (const matrix& l : g.leaves)
            if (l.storage->dev_stale) l.storage->upload();
        for (const matrix& n : g.order) {
            Primitive* p = n.tape.get();
            if (!p->is_view()) {
                p->stream = stream;
                p->execute(n);
            }
            p->evaluated = true;
            n.storage->dev_version++;
        }
    }
    std::vector<matrix> vjp(matrix&) override { throw std::logic_error("matrix: no vjp through a compiled graph"); }
    matrix jvp(std::vector<matrix>&) override { throw std::logic_error("matrix: no jvp through a compiled graph"); }
};

// The lazy nodes of one call: the inputs cast / packed to the placeholders' dtype and layout when
// they differ, one node per output sharing the output's buffer.
std::vector<matrix> call_subgraph(const std::shared_ptr<CompiledGraph>& g, const std::vector<matrix>& inputs) {
    if (inputs.size() != g->samples.size())
        throw std::invalid_argument("matrix: a compiled graph takes " + std::to_string(g->samples.size()) + " inputs, " +
                                    std::to_string(inputs.size()) + " given");
    std::vector<matrix> ins;
    for (size_t i = 0; i < inputs.size(); i++) {
        const matrix& x = inputs[i];
        const matrix& ph = g->samples[i];
        if (!x.storage || x.shape_vec() != ph.shape_vec())
            throw std::invalid_argument("matrix: a compiled graph's input shape differs from its sample's");
        const bool ok = x.type == ph.type && x.is_contiguous();
        ins.push_back(ok ? x : x.astype(ph.type, true));
    }
    auto prim = std::make_shared<CompiledNodePrim>(g, ins);
    std::vector<matrix> outs;
    for (const matrix& o : g->outputs)
        outs.push_back(matrix::make_view(o, o.shape_vec(), o.strides_vec(), o.offset, prim));
    return outs;
}

}  // namespace

std::function<matrix(const matrix&)> matrix::jit_graph_gpu(std::function<matrix(matrix)> func, matrix sample) {
    auto g = compile_subgraph({sample}, [&](std::vector<matrix> s) { return std::vector<matrix>{func(s[0])}; });
    return [g](const matrix& x) { return call_subgraph(g, {x})[0]; };
}

std::function<matrix(matrix)> matrix::grad_graph_gpu(std::function<matrix(matrix)> func, matrix sample) {
    auto g = compile_subgraph({sample}, [&](std::vector<matrix> s) {
        matrix out = func(s[0]);
        return std::vector<matrix>{build_grad_graph(out, s[0])};
    });
    return [g](matrix x) { return call_subgraph(g, {x})[0]; };
}

std::function<std::vector<matrix>(const std::vector<matrix>&)> matrix::multi_jit_graph_gpu(
    std::function<std::vector<matrix>(std::vector<matrix>)> func, const std::vector<matrix>& sample_inputs) {
    auto g = compile_subgraph(sample_inputs, func);
    return [g](const std::vector<matrix>& xs) { return call_subgraph(g, xs); };
}

std::function<std::vector<matrix>(std::vector<matrix>)> matrix::grad_graph_gpu(
    std::function<std::vector<matrix>(std::vector<matrix>)> func, const std::vector<matrix>& sample_inputs) {
    auto g = compile_subgraph(sample_inputs, [&](std::vector<matrix> s) {
        std::vector<matrix> outs = func(s);
        return build_grad_graph(outs, s);
    });
    return [g](std::vector<matrix> xs) { return call_subgraph(g, xs); };
}
