// reduce_ops.hpp -- reduction states shared by the reduction kernels and the fused
// broadcast-then-reduce kernel.  Semantics follow the reference CPU backends
// (Matrix.mm:15099-15208 sum, Matrix.mm:14812-15059 max / min, Matrix.mm:16182-16458 argmax /
// argmin): Max / Min start from dtype_lowest / dtype_max (matrix.h:271-282) and take a value only
// when strictly better, so NaN never wins and the first index wins among equals; every partial
// carries the index it came from and combine() breaks value ties by the smaller index.
#pragma once
#include "common.hpp"

#include <climits>
#include <cfloat>
#include <limits>

namespace mx {

constexpr uint32_t kEmpty = 0x7fffffffu;   // index of a partial that took no element

// ------------------------------------------------------------------ reduction states
template <typename T> __device__ __forceinline__ T shfl_x(T v, int m) { return __shfl_xor(v, m); }
template <> __device__ __forceinline__ uint8_t shfl_x(uint8_t v, int m) { return (uint8_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ int8_t shfl_x(int8_t v, int m) { return (int8_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ uint16_t shfl_x(uint16_t v, int m) { return (uint16_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ int16_t shfl_x(int16_t v, int m) { return (int16_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ uint32_t shfl_x(uint32_t v, int m) { return (uint32_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ uint64_t shfl_x(uint64_t v, int m) { return (uint64_t)__shfl_xor((long long)v, m); }
template <> __device__ __forceinline__ int64_t shfl_x(int64_t v, int m) { return (int64_t)__shfl_xor((long long)v, m); }

template <int DT> struct Limits {
    using C = typename dt_traits<DT>::C;
    __device__ __forceinline__ static C lowest() {
        if constexpr (DT == MX_FLOAT32) return -FLT_MAX;
        else if constexpr (DT == MX_FLOAT16) return -65504.0f;
        else if constexpr (DT == MX_BFLOAT16) return -3.38953138925153547590470800371487867e38f;  // -0x1.fep127
        else if constexpr (DT == MX_BOOL) return 0;
        else return std::numeric_limits<C>::lowest();
    }
    __device__ __forceinline__ static C highest() {
        if constexpr (DT == MX_FLOAT32) return FLT_MAX;
        else if constexpr (DT == MX_FLOAT16) return 65504.0f;
        else if constexpr (DT == MX_BFLOAT16) return 3.38953138925153547590470800371487867e38f;
        else if constexpr (DT == MX_BOOL) return 1;
        else return std::numeric_limits<C>::max();
    }
};

// Sum state: float for 16/32-bit floats, wrap-around unsigned for integers, OR for bool.
template <int DT> struct SumRed {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    using OutT = S;
    using St = std::conditional_t<Tr::is_float, float,
               std::conditional_t<(sizeof(S) <= 4), uint32_t, uint64_t>>;
    __device__ __forceinline__ static St init() { return St(0); }
    __device__ __forceinline__ static void step(St& s, S x, uint32_t) {
        if constexpr (Tr::is_float) s += Tr::ld(x);
        else if constexpr (DT == MX_BOOL) s |= (St)x;
        else s += (St)x;
    }
    __device__ __forceinline__ static St combine(St a, St b) {
        if constexpr (DT == MX_BOOL) return a | b;
        else return a + b;
    }
    __device__ __forceinline__ static St shfl(St a, int m) { return shfl_x(a, m); }
    __device__ __forceinline__ static OutT out(St s) {
        if constexpr (Tr::is_float) return Tr::st(s);
        else if constexpr (DT == MX_BOOL) return (OutT)(s != 0);
        else return (OutT)s;
    }
};

// (value, first index) state for Max / Min / ArgMax / ArgMin.
template <typename C> struct VI { C v; uint32_t i; };

template <int DT, bool IS_MAX, bool IS_ARG> struct ExtRed {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    using C = typename Tr::C;
    using OutT = std::conditional_t<IS_ARG, int32_t, S>;
    using St = VI<C>;
    __device__ __forceinline__ static bool better(C x, C cur) { return IS_MAX ? (cur < x) : (x < cur); }
    __device__ __forceinline__ static St init() {
        return St{IS_MAX ? Limits<DT>::lowest() : Limits<DT>::highest(), kEmpty};
    }
    __device__ __forceinline__ static void step(St& s, S x, uint32_t idx) {
        C v = Tr::ld(x);
        if (better(v, s.v)) { s.v = v; s.i = idx; }
    }
    __device__ __forceinline__ static St combine(St a, St b) {
        // b wins when strictly better, or equal and earlier (two empties keep a)
        bool take = better(b.v, a.v) || (!better(a.v, b.v) && b.i < a.i);
        return take ? b : a;
    }
    __device__ __forceinline__ static St shfl(St a, int m) {
        St r; r.v = shfl_x(a.v, m); r.i = shfl_x(a.i, m); return r;
    }
    __device__ __forceinline__ static OutT out(St s) {
        if constexpr (IS_ARG) return (int32_t)(s.i == kEmpty ? 0u : s.i);
        else {
            if (s.i == kEmpty) return Tr::st(IS_MAX ? Limits<DT>::lowest() : Limits<DT>::highest());
            return Tr::st(s.v);
        }
    }
};

template <int DT, int OP> struct RedSel;
template <int DT> struct RedSel<DT, MX_RED_SUM> { using R = SumRed<DT>; };
template <int DT> struct RedSel<DT, MX_RED_MAX> { using R = ExtRed<DT, true, false>; };
template <int DT> struct RedSel<DT, MX_RED_MIN> { using R = ExtRed<DT, false, false>; };
template <int DT> struct RedSel<DT, MX_RED_ARGMAX> { using R = ExtRed<DT, true, true>; };
template <int DT> struct RedSel<DT, MX_RED_ARGMIN> { using R = ExtRed<DT, false, true>; };

}  // namespace mx
