// common.hpp -- shared pieces of the gfx950 kernels and the C launch ABI.
//
// Element types are the reference's dtype codes (matrix.h:35-52).  16-bit floats are
// carried as raw uint16 bit patterns in memory and converted to float for arithmetic,
// which is what the reference's storage-only float16_t / bfloat16_t do on its CPU.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <string>
#include <type_traits>

#include "../../include/matrix_amd.h"

namespace mx {

// ------------------------------------------------------------------ errors
// Thread-local message for mx_last_error(); every ABI entry point returns a status.
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int hip_fail(hipError_t err, const char* what);

#define MX_HIP(call)                                                   \
    do {                                                               \
        hipError_t e_ = (call);                                        \
        if (e_ != hipSuccess) return ::mx::hip_fail(e_, #call);        \
    } while (0)

// Resolves a NULL stream to the calling thread's stream.  Returns false (with the error
// set) when the runtime was never initialised.
bool resolve_stream(void* in, hipStream_t* out);


// ------------------------------------------------------------------ element types
struct half_bits { uint16_t v; };   // IEEE binary16, stored raw
struct bf16_bits { uint16_t v; };   // bfloat16, stored raw

__device__ __forceinline__ float bits_to_float(uint16_t h) {
    _Float16 x = __builtin_bit_cast(_Float16, h);
    return (float)x;
}
// Round-to-nearest-even float -> half (v_cvt_f16_f32 honours the default RNE mode).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    _Float16 x = (_Float16)f;
    return __builtin_bit_cast(uint16_t, x);
}
__device__ __forceinline__ float bf16_to_float(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}
// Round-to-nearest-even float -> bfloat16; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t float_to_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Traits: storage type S, compute type C, load/store between them.
template <int DT> struct dt_traits;
#define MX_INT_TRAITS(CODE, TYPE)                                                   \
    template <> struct dt_traits<CODE> {                                            \
        using S = TYPE; using C = TYPE;                                             \
        static constexpr bool is_float = false;                                     \
        static constexpr bool is_signed = std::is_signed<TYPE>::value;              \
        __device__ __forceinline__ static C ld(S x) { return x; }                   \
        __device__ __forceinline__ static S st(C x) { return x; }                   \
    };
MX_INT_TRAITS(MX_UINT8, uint8_t)
MX_INT_TRAITS(MX_INT32, int32_t)
MX_INT_TRAITS(MX_INT16, int16_t)
MX_INT_TRAITS(MX_UINT32, uint32_t)
MX_INT_TRAITS(MX_UINT16, uint16_t)
MX_INT_TRAITS(MX_INT8, int8_t)
MX_INT_TRAITS(MX_INT64, int64_t)
MX_INT_TRAITS(MX_UINT64, uint64_t)
#undef MX_INT_TRAITS
template <> struct dt_traits<MX_BOOL> {           // bool stored as one byte 0 / 1
    using S = uint8_t; using C = uint8_t;
    static constexpr bool is_float = false;
    static constexpr bool is_signed = false;
    __device__ __forceinline__ static C ld(S x) { return x; }
    __device__ __forceinline__ static S st(C x) { return x; }
};
template <> struct dt_traits<MX_FLOAT32> {
    using S = float; using C = float;
    static constexpr bool is_float = true;
    static constexpr bool is_signed = true;
    __device__ __forceinline__ static C ld(S x) { return x; }
    __device__ __forceinline__ static S st(C x) { return x; }
};
template <> struct dt_traits<MX_FLOAT16> {
    using S = uint16_t; using C = float;
    static constexpr bool is_float = true;
    static constexpr bool is_signed = true;
    __device__ __forceinline__ static C ld(S x) { return bits_to_float(x); }
    __device__ __forceinline__ static S st(C x) { return float_to_half_bits(x); }
};
template <> struct dt_traits<MX_BFLOAT16> {
    using S = uint16_t; using C = float;
    static constexpr bool is_float = true;
    static constexpr bool is_signed = true;
    __device__ __forceinline__ static C ld(S x) { return bf16_to_float(x); }
    __device__ __forceinline__ static S st(C x) { return float_to_bf16(x); }
};

// complex64 (type code 9, complex.h:18-26): two floats, re first, 8-byte aligned (numpy's
// complex64, float2).
struct alignas(8) c64 { float re, im; };
template <> struct dt_traits<MX_COMPLEX64> {
    using S = c64; using C = c64;
    static constexpr bool is_float = false;
    static constexpr bool is_signed = true;
    __device__ __forceinline__ static C ld(S x) { return x; }
    __device__ __forceinline__ static S st(C x) { return x; }
};

inline size_t dtype_size(int dt) {
    switch (dt) {
    case MX_FLOAT32: case MX_INT32: case MX_UINT32: return 4;
    case MX_FLOAT16: case MX_INT16: case MX_UINT16: case MX_BFLOAT16: return 2;
    case MX_UINT8: case MX_INT8: case MX_BOOL: return 1;
    case MX_INT64: case MX_UINT64: case MX_COMPLEX64: return 8;
    default: return 0;
    }
}

// Calls f(std::integral_constant<int, DT>{}) for the 12 real dtypes; false for others.
template <typename F>
inline bool dispatch_dtype(int dt, F&& f) {
    switch (dt) {
    case MX_FLOAT32: f(std::integral_constant<int, MX_FLOAT32>{}); return true;
    case MX_FLOAT16: f(std::integral_constant<int, MX_FLOAT16>{}); return true;
    case MX_BFLOAT16: f(std::integral_constant<int, MX_BFLOAT16>{}); return true;
    case MX_UINT8: f(std::integral_constant<int, MX_UINT8>{}); return true;
    case MX_INT32: f(std::integral_constant<int, MX_INT32>{}); return true;
    case MX_INT16: f(std::integral_constant<int, MX_INT16>{}); return true;
    case MX_UINT32: f(std::integral_constant<int, MX_UINT32>{}); return true;
    case MX_UINT16: f(std::integral_constant<int, MX_UINT16>{}); return true;
    case MX_BOOL: f(std::integral_constant<int, MX_BOOL>{}); return true;
    case MX_INT8: f(std::integral_constant<int, MX_INT8>{}); return true;
    case MX_INT64: f(std::integral_constant<int, MX_INT64>{}); return true;
    case MX_UINT64: f(std::integral_constant<int, MX_UINT64>{}); return true;
    default: return false;
    }
}

// ------------------------------------------------------------------ fast division
// Unsigned division by a runtime-constant divisor with one mul-hi and a shift
// (Granlund & Montgomery, "Division by invariant integers using multiplication", 1994):
// for d > 0, s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1, n / d = (mulhi(n, m) + n) >> s
// for every 32-bit n (the add is done in 64 bits).
struct FastDiv {
    uint32_t d = 1, m = 0, s = 0;
    FastDiv() = default;
    explicit FastDiv(uint32_t div) : d(div) {
        s = 0;
        while (s < 32 && (1ull << s) < div) s++;
        m = (uint32_t)((((1ull << 32) * ((1ull << s) - div)) / div) + 1);
    }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
        uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
        return (uint32_t)(((uint64_t)hi + n) >> s);
    }
};

// Small-array descriptors passed by value as kernel arguments.
template <int N>
struct DimArr {
    uint32_t v[N];
};

// Nontemporal (streaming) load of one 4-, 8- or 16-byte value, for inputs that are read once by
// load instructions that each cover whole 128-byte lines; other sizes load normally.
template <class V>
__device__ __forceinline__ V ld_stream(const V* p) {
    if constexpr (sizeof(V) == 16) {
        using U = unsigned __attribute__((ext_vector_type(4)));
        return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const U*>(p)));
    } else if constexpr (sizeof(V) == 8) {
        using U = unsigned __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const U*>(p)));
    } else if constexpr (sizeof(V) == 4) {
        return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(p)));
    } else {
        return *p;
    }
}

}  // namespace mx
