// matrix.hpp -- the lazy-graph matrix API of the GPU evaluation path, over the gfx950 launch ABI.
//
// API-compatible subset of the reference's matrix / Primitive layer for the hot path (matrix.h:
// 496-1771, primitives.cpp:57-118): building ops records Primitive nodes on a tape; eval()
// compiles and runs the graph; compile_gpu() / execute_gpu() / clear_trace_checks() are the
// compile-once, execute-many cycle of compile_metal / execute_metal (Matrix.mm:8452-8475); vjp and
// build_grad_graph / value_and_grad are the reverse-mode autodiff of Matrix.mm:1177-1411.
//
// What differs from the reference, by design:
//   - data live in device memory (HBM); a leaf keeps a host copy that is uploaded at compile
//     time and again after mark_changed(); to_host() downloads;
//   - every Primitive's eval runs on the gfx950 kernels; there is no CPU evaluation path;
//   - compile allocates every node's output and workspace; execute never allocates (the
//     reference's law, .agents/MemoryManagement.md:24), and queues all launches on the calling
//     thread's stream with a single wait at the end.
#pragma once

#include <complex>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

// dtype codes of matrix.h:35-52
enum class dtype : uint8_t {
    Float = 0, Float16 = 1, UInt8 = 2, Int32 = 3, Int16 = 4, UInt32 = 5, UInt16 = 6,
    Bool = 7, Int8 = 8, Complex64 = 9, BFloat16 = 10, Int64 = 11, UInt64 = 12
};
using size_m = uint32_t;

size_t dtype_size(dtype t);
const char* dtype_name(dtype t);

constexpr bool is_complex(dtype d) { return d == dtype::Complex64; }
constexpr bool is_floating(dtype d) { return d == dtype::Float || d == dtype::Float16 || d == dtype::BFloat16; }
constexpr bool is_integral(dtype d) { return !is_floating(d) && !is_complex(d) && d != dtype::Bool; }
constexpr bool is_unsigned(dtype d) {
    return d == dtype::UInt8 || d == dtype::UInt16 || d == dtype::UInt32 || d == dtype::UInt64;
}

// The dtype of a binary op's result (type_rules / promote_types, matrix.h:166-180,
// Matrix.mm:107-109): Complex64 absorbs everything; Bool takes the other dtype; Float absorbs
// the rest; a 16-bit float with anything but itself or Bool is Float; two integers of one
// signedness take the wider; a signed and an unsigned integer take the signed one when it is
// wider, else Float next to UInt64, else the signed type twice the unsigned's width (at most
// Int32).
dtype promote_types(dtype a, dtype b);

template <typename T> constexpr dtype dtype_of() {
    if constexpr (std::is_same_v<T, float>) return dtype::Float;
    else if constexpr (std::is_same_v<T, int32_t>) return dtype::Int32;
    else if constexpr (std::is_same_v<T, int64_t>) return dtype::Int64;
    else if constexpr (std::is_same_v<T, uint32_t>) return dtype::UInt32;
    else if constexpr (std::is_same_v<T, uint64_t>) return dtype::UInt64;
    else if constexpr (std::is_same_v<T, int16_t>) return dtype::Int16;
    else if constexpr (std::is_same_v<T, uint16_t>) return dtype::UInt16;
    else if constexpr (std::is_same_v<T, int8_t>) return dtype::Int8;
    else if constexpr (std::is_same_v<T, uint8_t>) return dtype::UInt8;
    else if constexpr (std::is_same_v<T, bool>) return dtype::Bool;
    else if constexpr (std::is_same_v<T, double>) return dtype::Float;
    else if constexpr (std::is_same_v<T, int>) return dtype::Int32;
    else if constexpr (std::is_same_v<T, _Float16>) return dtype::Float16;
    else if constexpr (std::is_same_v<T, __bf16>) return dtype::BFloat16;
    else if constexpr (std::is_same_v<T, std::complex<float>>) return dtype::Complex64;
    else static_assert(sizeof(T) == 0, "no dtype for this C++ type");
}

namespace matrix_amd {
// Device residency of one allocation (shared by a node's output and every view of it).
struct Storage {
    size_t bytes = 0;
    void* dev = nullptr;
    std::vector<uint8_t> host;        // a leaf's values (host side); a node's at() cache
    bool host_is_source = false;      // leaf: host holds the values, device gets a copy
    bool dev_stale = true;            // host changed since the last upload
    bool borrowed = false;            // dev points into another allocation (a compiled graph's input)
    uint64_t dev_version = 0;         // bumped by every execute that writes the device copy
    uint64_t leaf_version = 0;        // a leaf's version: the epoch of its last mark_changed()
    uint64_t host_version = ~0ull;    // dev_version the host cache of a node holds
    ~Storage();
    void allocate();                  // device memory of `bytes` (once)
    void upload();                    // host -> device, synchronous
};
// Initialises the device on first use (device 0 unless init() chose another).
void init(int device = 0);
}  // namespace matrix_amd

class Primitive;

class matrix {
public:
    uint32_t dims = 0;
    dtype type = dtype::Float;
    std::shared_ptr<Primitive> tape;                   // null for a leaf
    std::shared_ptr<matrix_amd::Storage> storage;
    size_t offset = 0;                                 // element offset of this view

    matrix() = default;

    // ---- shape
    size_m* shape() { return shp_.data(); }
    const size_m* shape() const { return shp_.data(); }
    size_m* strides() { return str_.data(); }
    const size_m* strides() const { return str_.data(); }
    std::vector<size_m> shape_vec() const { return shp_; }
    std::vector<size_m> strides_vec() const { return str_; }
    size_t total_size() const;
    bool is_contiguous() const;

    // ---- creation (leaves)
    static matrix leaf(const std::vector<size_m>& shape, dtype type = dtype::Float);
    static matrix leaf(std::initializer_list<size_m> shape, dtype type = dtype::Float) {
        return leaf(std::vector<size_m>(shape), type);
    }
    static matrix from_bytes(const std::vector<size_m>& shape, dtype type, const void* data);
    template <typename T>
    static matrix from_host(const std::vector<size_m>& shape, const std::vector<T>& data, dtype type = dtype_of<T>()) {
        if (dtype_size(type) != sizeof(T)) throw std::invalid_argument("matrix::from_host: element size mismatch");
        return from_bytes(shape, type, data.data());
    }
    // A rank-0 matrix holding val converted to type (matrix.h:648-660: static_cast, the 16-bit
    // floats rounded to nearest even).  The 16-bit float types are listed on their own: the
    // standard library does not count them as arithmetic.
    template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T> || std::is_same_v<T, _Float16> ||
                                                      std::is_same_v<T, __bf16>>>
    static matrix scalar(T val, dtype type = dtype_of<T>()) {
        matrix m = leaf({}, type);
        store_scalar(type, val, m.host_data());
        return m;
    }
    static matrix full(const std::vector<size_m>& shape, double value, dtype type = dtype::Float);
    static matrix zeros(const std::vector<size_m>& shape, dtype type = dtype::Float) { return full(shape, 0.0, type); }
    static matrix ones(const std::vector<size_m>& shape, dtype type = dtype::Float) { return full(shape, 1.0, type); }
    matrix zeros() const { return zeros(shp_, type); }
    matrix ones() const { return ones(shp_, type); }
    void* host_data();               // a leaf's host values (write, then mark_changed())
    void mark_changed();
    // A one-element leaf holding value (matrix.h:917): the tracked scalar a caller writes into
    // (host_data / at), then mark_changed(), and the next execute sees it.
    static matrix leaf_scalar(float value, dtype type = dtype::Float);
    // Evaluate, then keep the values and drop the graph: the matrix becomes a leaf whose data stay
    // on the device (make_leaf, Matrix.mm:2686-2691; releaseTape drops the graph of an evaluated
    // node the same way).
    void make_leaf();
    void releaseTape();

    // ---- views and casts
    matrix transpose(const std::vector<size_m>& order) const;
    matrix reshape(const std::vector<size_m>& new_shape) const;
    matrix flatten(int start, int end) const;
    matrix unsqueeze(int axis) const;
    matrix broadcast_to(const std::vector<size_m>& shape) const;
    matrix astype(dtype t, bool make_contig = false) const;

    // ---- element-wise (broadcasting, Matrix.mm:161-232)
    friend matrix operator+(const matrix& a, const matrix& b);
    friend matrix operator-(const matrix& a, const matrix& b);
    friend matrix operator*(const matrix& a, const matrix& b);
    friend matrix operator/(const matrix& a, const matrix& b);
    static matrix max(const matrix& a, const matrix& b);
    static matrix min(const matrix& a, const matrix& b);
    static matrix equal(const matrix& a, const matrix& b);

    // ---- reductions (one axis, Matrix.mm:14784-16458)
    matrix sum(int axis, bool keepdims = false) const;
    matrix sum(int start, int end, bool keepdims) const;
    matrix sum() const;
    matrix max(int axis, bool keepdims = false) const;
    matrix min(int axis, bool keepdims = false) const;
    matrix argmax(int axis, bool keepdims = false) const;
    matrix argmin(int axis, bool keepdims = false) const;
    matrix SumNoRed(int axis) const;                    // sum keeping the axis (extent 1)
    matrix unbroadcast_shape(const size_m* target_shape, int target_dims) const;

    // ---- contractions
    matrix dot(const matrix& b, bool transposeB = false) const;
    static matrix conv(const matrix& input, const matrix& kernel, const std::vector<int>& stride,
                       const std::vector<int>& pad_lo, const std::vector<int>& pad_hi,
                       const std::vector<int>& kernel_dilation, const std::vector<int>& input_dilation,
                       int groups = 1, bool flip = false);
    static matrix conv2d(const matrix& input, const matrix& kernel, int stride_h = 1, int stride_w = 1,
                         int pad_h = 0, int pad_w = 0, int dilation_h = 1, int dilation_w = 1, int groups = 1,
                         int input_dilation_h = 1, int input_dilation_w = 1, bool flip = false);

    // ---- files
    // One uncompressed .npy per matrix (arr_0.npy, arr_1.npy, ...) in a STORED ZIP, byte for byte as
    // the reference writes it (Matrix.mm:3748-4085, matrix.h:1237); evaluates each matrix first.
    static void save_as_npz(std::vector<matrix> input, std::string file_path);
    // Reads an .npz of STORED entries (save_as_npz's, or np.savez's) into host leaves, in archive
    // order; names (optional) receives each entry's name without ".npy".  No reference counterpart.
    static std::vector<matrix> load_npz(const std::string& file_path, std::vector<std::string>* names = nullptr);

    // ---- evaluation
    void eval();
    void compile_gpu();
    void execute_gpu();
    void clear_trace_checks();
    static void eval(std::vector<matrix>& ms);
    static void compile_gpu(std::vector<matrix>& ms);
    static void execute_gpu(std::vector<matrix>& ms);
    static void clear_trace_checks(std::vector<matrix>& ms);
    std::vector<uint8_t> to_host_bytes() const;       // values in row-major order (evaluates)
    template <typename T> std::vector<T> to_host() const {
        if (dtype_size(type) != sizeof(T)) throw std::invalid_argument("matrix::to_host: element size mismatch");
        std::vector<uint8_t> b = to_host_bytes();
        std::vector<T> out(b.size() / sizeof(T));
        if (!b.empty()) std::memcpy(out.data(), b.data(), b.size());
        return out;
    }

    // The reference's names for the same cycle (Matrix.mm:8436-8469): compile_metal allocates,
    // execute_metal launches and waits, eval_metal does both.  The device is the MI355X.
    void compile_metal() { compile_gpu(); }
    void execute_metal() { execute_gpu(); }
    void eval_metal() { eval(); }
    // Several at once (matrix.h:1722-1729): each argument a matrix or a std::vector<matrix>; one
    // execute for all of them.  detach drops each one's graph and keeps its data.
    template <typename... Args> static void eval(Args&... args) {
        std::vector<matrix> all;
        (gather(all, args), ...);
        eval(all);
    }
    template <typename... Args> static void detach(Args&... args) { (detach_each(args), ...); }
    // Element access (matrix.h:1734-1764): evaluates when needed, checks the rank, the dtype and
    // every index, and returns a reference to the element in a host copy of the values (a leaf's
    // own host values: write through it, then mark_changed(), as the reference requires).
    template <typename T, typename... Args> T& at(Args... args) {
        constexpr size_t N = sizeof...(args);
        if (dims != N) throw std::runtime_error("Matrix rank mismatch in at().");
        if (type != dtype_of<T>()) throw std::runtime_error("Type mismatch in at().");
        size_t off = offset;
        if constexpr (N > 0) {
            const size_m idx[N] = {static_cast<size_m>(args)...};
            for (size_t d = 0; d < N; ++d) {
                if (idx[d] >= shp_[d])
                    throw std::out_of_range("at(): index " + std::to_string(idx[d]) + " out of bounds for dimension " +
                                            std::to_string(d) + " with shape " + std::to_string(shp_[d]));
                off += (size_t)idx[d] * str_[d];
            }
        }
        return reinterpret_cast<T*>(host_view())[off];
    }

    // ---- autodiff
    static std::vector<matrix> build_grad_graph(std::vector<matrix>& output_nodes,
                                                std::vector<matrix>& sample_input_nodes);
    static matrix build_grad_graph(matrix& output_node, matrix& sample_input_node);
    static std::function<std::pair<matrix, std::vector<matrix>>(const std::vector<matrix>&)> value_and_grad(
        std::function<matrix(std::vector<matrix>)> fn);
    static std::function<std::pair<matrix, matrix>(const matrix&)> value_and_grad(std::function<matrix(matrix)> fn);
    static std::function<std::vector<matrix>(const std::vector<matrix>&)> grad(
        std::function<matrix(std::vector<matrix>)> fn);
    static std::function<matrix(const matrix&)> grad(std::function<matrix(matrix)> fn);
    // Forward mode (no counterpart in the reference, which has the per-node jvp only,
    // primitives.cpp:110): the tangent of every output for the given tangents of the inputs, built
    // from each node's jvp in topological order (inputs without a tangent contribute zero).
    static std::vector<matrix> build_jvp_graph(std::vector<matrix>& output_nodes, std::vector<matrix>& input_nodes,
                                               std::vector<matrix>& input_tangents);

    // ---- compiled sub-graphs (Matrix.mm:1076-1175, 1413-1470): func is traced once on a leaf of
    // the sample's shape and dtype and compiled; each call of the returned function gives lazy
    // nodes that run the compiled graph on the call's inputs (no copy of them: the graph reads
    // their buffers) and share its output buffers, as the reference's do.
    static std::function<matrix(const matrix&)> jit_graph_gpu(std::function<matrix(matrix)> func, matrix sample);
    static std::function<matrix(matrix)> grad_graph_gpu(std::function<matrix(matrix)> func, matrix sample);
    static std::function<std::vector<matrix>(const std::vector<matrix>&)> multi_jit_graph_gpu(
        std::function<std::vector<matrix>(std::vector<matrix>)> func, const std::vector<matrix>& sample_inputs);
    static std::function<std::vector<matrix>(std::vector<matrix>)> grad_graph_gpu(
        std::function<std::vector<matrix>(std::vector<matrix>)> func, const std::vector<matrix>& sample_inputs);

    // (internal) a node's output handle
    static matrix make_node(std::vector<size_m> shape, dtype type, std::shared_ptr<Primitive> prim);
    static matrix make_view(const matrix& base, std::vector<size_m> shape, std::vector<size_m> strides,
                            size_t offset, std::shared_ptr<Primitive> prim);
    void* device_ptr() const;                          // valid after compile

private:
    std::vector<size_m> shp_, str_;
    friend class Primitive;
    void* host_view();                 // host copy of the storage (evaluates, downloads when stale)
    static void gather(std::vector<matrix>& all, matrix& m) { all.push_back(m); }
    static void gather(std::vector<matrix>& all, std::vector<matrix>& ms) { all.insert(all.end(), ms.begin(), ms.end()); }
    static void detach_each(matrix& m) { m.releaseTape(); }
    static void detach_each(std::vector<matrix>& ms) { for (auto& m : ms) m.releaseTape(); }
    template <typename T> static void store_scalar(dtype type, T val, void* dst);
};

template <typename T>
void matrix::store_scalar(dtype type, T v, void* dst) {
    auto put = [dst](auto x) { std::memcpy(dst, &x, sizeof(x)); };
    switch (type) {
    case dtype::Float: put(static_cast<float>(v)); break;
    case dtype::Float16: put(static_cast<_Float16>(v)); break;
    case dtype::BFloat16: put(static_cast<__bf16>(static_cast<float>(v))); break;
    case dtype::Int8: put(static_cast<int8_t>(v)); break;
    case dtype::UInt8: put(static_cast<uint8_t>(v)); break;
    case dtype::Bool: put(static_cast<uint8_t>(v != T(0))); break;
    case dtype::Int16: put(static_cast<int16_t>(v)); break;
    case dtype::UInt16: put(static_cast<uint16_t>(v)); break;
    case dtype::Int32: put(static_cast<int32_t>(v)); break;
    case dtype::UInt32: put(static_cast<uint32_t>(v)); break;
    case dtype::Int64: put(static_cast<int64_t>(v)); break;
    case dtype::UInt64: put(static_cast<uint64_t>(v)); break;
    case dtype::Complex64: { float c[2] = {static_cast<float>(v), 0.0f}; std::memcpy(dst, c, 8); break; }
    }
}

// The dtype a C++ scalar takes next to a matrix of dtype m (scalar_operand_type,
// matrix.h:1815-1840): m itself whenever that holds the value, so the scalar never widens the
// matrix (uint8 * 2 stays uint8, half * 0.5f stays Float16), otherwise the narrowest dtype that
// does and that promote_types then settles on:
//   - m Float / BFloat16 / Complex64, or a bool scalar: m;
//   - m Float16: m within +-65504, else Float;
//   - a floating-point scalar next to an integer (or Bool) matrix: Float;
//   - an integer scalar: m if it fits, else Int32, else UInt32 (m unsigned), else Int64
//     (m not UInt64), else UInt64 (m unsigned); std::overflow_error when none holds it.
namespace matrix_amd_detail {
template <typename T>
constexpr bool in_range(T v, long double lo, long double hi) {
    if constexpr (std::is_floating_point_v<T>) return v >= (T)lo && v <= (T)hi;
    else if constexpr (std::is_signed_v<T>) return (long double)v >= lo && (long double)v <= hi;
    else return (long double)v <= hi;
}
}  // namespace matrix_amd_detail

template <typename T>
dtype scalar_operand_type(T v, dtype m) {
    static_assert(std::is_arithmetic_v<T>, "matrix op with a non-arithmetic scalar");
    using matrix_amd_detail::in_range;
    if (m == dtype::Float || m == dtype::BFloat16 || m == dtype::Complex64) return m;
    if constexpr (std::is_same_v<T, bool>) return m;
    if (m == dtype::Float16) return in_range(v, -65504.0L, 65504.0L) ? m : dtype::Float;
    if constexpr (std::is_floating_point_v<T>) {
        return dtype::Float;
    } else {
        auto holds = [&](dtype d) -> bool {
            switch (d) {
            case dtype::Int8: return in_range(v, -128.0L, 127.0L);
            case dtype::UInt8: return in_range(v, 0.0L, 255.0L);
            case dtype::Int16: return in_range(v, -32768.0L, 32767.0L);
            case dtype::UInt16: return in_range(v, 0.0L, 65535.0L);
            case dtype::Int32: return in_range(v, -2147483648.0L, 2147483647.0L);
            case dtype::UInt32: return in_range(v, 0.0L, 4294967295.0L);
            case dtype::Int64: return in_range(v, -9223372036854775808.0L, 9223372036854775807.0L);
            case dtype::UInt64: if constexpr (std::is_signed_v<T>) return v >= 0; else return true;
            default: return false;
            }
        };
        if (holds(m)) return m;                  // Bool holds no integer scalar: Int32 next
        if (holds(dtype::Int32)) return dtype::Int32;
        const bool mu = is_unsigned(m);
        if (mu && holds(dtype::UInt32)) return dtype::UInt32;
        if (m != dtype::UInt64 && holds(dtype::Int64)) return dtype::Int64;
        if (mu && holds(dtype::UInt64)) return dtype::UInt64;
        throw std::overflow_error("matrix op: scalar " + std::to_string(v) +
                                  " doesn't fit any dtype it could promote to");
    }
}

// matrix (op) scalar and scalar (op) matrix: the scalar becomes a rank-0 matrix of
// scalar_operand_type(scalar, m.type) and the matrix operator promotes (matrix.h:1842-1870).
#define MATRIX_AMD_SCALAR_OP(OP)                                                              \
    template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>              \
    inline matrix operator OP(const matrix& m, T v) {                                        \
        return m OP matrix::scalar(v, scalar_operand_type(v, m.type));                       \
    }                                                                                         \
    template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>              \
    inline matrix operator OP(T v, const matrix& m) {                                        \
        return matrix::scalar(v, scalar_operand_type(v, m.type)) OP m;                       \
    }
MATRIX_AMD_SCALAR_OP(+)
MATRIX_AMD_SCALAR_OP(-)
MATRIX_AMD_SCALAR_OP(*)
MATRIX_AMD_SCALAR_OP(/)
#undef MATRIX_AMD_SCALAR_OP

// A node of the graph: the reference's Primitive contract (primitives.cpp:57-118).  compile()
// prepares descriptors and workspace once; execute() only launches; vjp() builds the gradient
// graph of its inputs.
class Primitive {
public:
    virtual ~Primitive() = default;
    virtual const char* name() const = 0;
    virtual uint32_t num_inputs() const = 0;
    virtual matrix& input_at(uint32_t i) = 0;
    virtual bool is_view() const { return false; }
    virtual void compile(const matrix& out) = 0;
    virtual void execute(const matrix& out) = 0;
    virtual std::vector<matrix> vjp(matrix& grad_out) = 0;
    // The tangent of this node's output from the tangents of its inputs (primitives.cpp:110).
    virtual matrix jvp(std::vector<matrix>& tangents) = 0;
    // Copies of the input handles, in input_at order (primitives.cpp:112).
    std::vector<matrix> get_inputs() {
        std::vector<matrix> v;
        for (uint32_t i = 0; i < num_inputs(); i++) v.push_back(input_at(i));
        return v;
    }
    // Re-evaluation after leaves change (primitives.cpp:117): a node is invalidated (evaluated =
    // false) when any input is, or when an input leaf was marked changed after this node last
    // took its version; memoised per pass.  Returns whether the node must run again.
    bool invalidate_pass(uint64_t current_pass_id);
    bool compiled = false;
    bool evaluated = false;
    uint64_t version = 1;
    uint64_t last_visited_pass_id = 0;
    void* stream = nullptr;        // the stream execute() launches on (set by the executor)
    uint64_t run_gen = 0;          // the executing thread's execute count when this node was scheduled
};
