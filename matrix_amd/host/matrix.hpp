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
    else static_assert(sizeof(T) == 0, "no dtype for this C++ type");
}

namespace matrix_amd {
// Device residency of one allocation (shared by a node's output and every view of it).
struct Storage {
    size_t bytes = 0;
    void* dev = nullptr;
    std::vector<uint8_t> host;        // a leaf's values (host side)
    bool host_is_source = false;      // leaf: host holds the values, device gets a copy
    bool dev_stale = true;            // host changed since the last upload
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
    static matrix scalar(double value, dtype type = dtype::Float);
    static matrix full(const std::vector<size_m>& shape, double value, dtype type = dtype::Float);
    static matrix zeros(const std::vector<size_m>& shape, dtype type = dtype::Float) { return full(shape, 0.0, type); }
    static matrix ones(const std::vector<size_m>& shape, dtype type = dtype::Float) { return full(shape, 1.0, type); }
    matrix zeros() const { return zeros(shp_, type); }
    matrix ones() const { return ones(shp_, type); }
    void* host_data();               // a leaf's host values (write, then mark_changed())
    void mark_changed();

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

    // ---- autodiff
    static std::vector<matrix> build_grad_graph(std::vector<matrix>& output_nodes,
                                                std::vector<matrix>& sample_input_nodes);
    static matrix build_grad_graph(matrix& output_node, matrix& sample_input_node);
    static std::function<std::pair<matrix, std::vector<matrix>>(const std::vector<matrix>&)> value_and_grad(
        std::function<matrix(std::vector<matrix>)> fn);
    static std::function<std::vector<matrix>(const std::vector<matrix>&)> grad(
        std::function<matrix(std::vector<matrix>)> fn);

    // (internal) a node's output handle
    static matrix make_node(std::vector<size_m> shape, dtype type, std::shared_ptr<Primitive> prim);
    static matrix make_view(const matrix& base, std::vector<size_m> shape, std::vector<size_m> strides,
                            size_t offset, std::shared_ptr<Primitive> prim);
    void* device_ptr() const;                          // valid after compile

private:
    std::vector<size_m> shp_, str_;
    friend class Primitive;
};

// Scalars on either side take the matrix's dtype (scalar_operand_type, matrix.h:494).
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator+(const matrix& a, T v) { return a + matrix::scalar((double)v, a.type); }
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator+(T v, const matrix& a) { return matrix::scalar((double)v, a.type) + a; }
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator-(const matrix& a, T v) { return a - matrix::scalar((double)v, a.type); }
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator-(T v, const matrix& a) { return matrix::scalar((double)v, a.type) - a; }
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator*(const matrix& a, T v) { return a * matrix::scalar((double)v, a.type); }
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator*(T v, const matrix& a) { return matrix::scalar((double)v, a.type) * a; }
template <typename T, typename = std::enable_if_t<std::is_arithmetic_v<T>>>
inline matrix operator/(const matrix& a, T v) { return a / matrix::scalar((double)v, a.type); }

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
    bool compiled = false;
    bool evaluated = false;
    void* stream = nullptr;        // the stream execute() launches on (set by the executor)
};
