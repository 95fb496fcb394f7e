// elementwise.hpp -- the per-element binary operations of the broadcast kernels (Add / Sub /
// Mul / Divide / Max / Min / Equal), shared by the broadcast kernel and the fused
// broadcast-then-reduce kernel.  Semantics follow the reference CPU backends
// (Matrix.mm:7411-7707, Matrix.mm:13378-13478, Matrix.mm:14668-14783, Matrix.mm:14469-14540):
// 16-bit floats compute in float and round once; integers wrap; integer division truncates, a
// zero divisor gives 0 and MIN / -1 gives MIN (arm64); Max is (a < b) ? b : a and Min is
// (b < a) ? b : a on the operands' own bits; Equal writes 1 / 0 in the operands' dtype.
// complex64 has Add / Sub / Mul / Divide only (the reference instantiates its broadcast
// kernels for type 9 in those four, BrodcastedMul.metal:95), with complex.h's arithmetic:
//   (a + bi) +- (c + di) = (a +- c) + (b +- d)i;
//   (a + bi)(c + di) = (a, b) c + (-b, a) d (complex.h:36-38), which clang's default contraction
//     (-ffp-contract=on) makes one rounded product and one fused multiply-add per part:
//     re = fma(a, c, -(b d)), im = fma(b, c, a d);
//   (a + bi) / (c + di) = ((a + bi)(c - di)) / (c c + d d) (complex.h:40-52): the product as
//     above with conj(rhs) = (c, -d), then both parts divided (IEEE) by c c + d d, whose two
//     squares are each rounded (simd_length_squared sums outside the expression).  No scaling:
//     |rhs| beyond ~1.8e19 overflows c c + d d, as in the reference.
#pragma once
#include "common.hpp"

namespace mx {

template <int DT, int OP>
struct BinOp {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    __device__ __forceinline__ static S apply(S a, S b) {
        if constexpr (DT == MX_COMPLEX64) {
#pragma clang fp contract(off)
            static_assert(OP == MX_OP_ADD || OP == MX_OP_SUB || OP == MX_OP_MUL || OP == MX_OP_DIV,
                          "complex64: Add / Sub / Mul / Divide only");
            if constexpr (OP == MX_OP_ADD) return c64{a.re + b.re, a.im + b.im};
            else if constexpr (OP == MX_OP_SUB) return c64{a.re - b.re, a.im - b.im};
            else if constexpr (OP == MX_OP_MUL) return c64{__builtin_fmaf(a.re, b.re, -(a.im * b.im)),
                                                           __builtin_fmaf(a.im, b.re, a.re * b.im)};
            else {
                const float c = b.re, d = -b.im;                 // conj(rhs)
                const float re = __builtin_fmaf(a.re, c, -(a.im * d));
                const float im = __builtin_fmaf(a.im, c, a.re * d);
                const float m = b.re * b.re + b.im * b.im;
                return c64{re / m, im / m};
            }
        } else if constexpr (Tr::is_float) {
            float x = Tr::ld(a), y = Tr::ld(b);
            if constexpr (OP == MX_OP_ADD) return Tr::st(x + y);
            else if constexpr (OP == MX_OP_SUB) return Tr::st(x - y);
            else if constexpr (OP == MX_OP_MUL) return Tr::st(x * y);
            else if constexpr (OP == MX_OP_DIV) return Tr::st(x / y);
            else if constexpr (OP == MX_OP_MAX) return (x < y) ? b : a;
            else if constexpr (OP == MX_OP_MIN) return (y < x) ? b : a;
            else return (x == y) ? Tr::st(1.0f) : Tr::st(0.0f);
        } else if constexpr (DT == MX_BOOL) {
            int x = a, y = b;
            if constexpr (OP == MX_OP_ADD) return (S)((x + y) != 0);
            else if constexpr (OP == MX_OP_SUB) return (S)((x - y) != 0);
            else if constexpr (OP == MX_OP_MUL) return (S)((x * y) != 0);
            else if constexpr (OP == MX_OP_DIV) return (S)(y == 0 ? 0 : ((x / y) != 0));
            else if constexpr (OP == MX_OP_MAX) return (x < y) ? b : a;
            else if constexpr (OP == MX_OP_MIN) return (y < x) ? b : a;
            else return (S)(x == y ? 1 : 0);
        } else {
            // wrap-around arithmetic in an unsigned type at least 32 bits wide
            using U = std::conditional_t<(sizeof(S) <= 4), uint32_t, uint64_t>;
            if constexpr (OP == MX_OP_ADD) return (S)((U)a + (U)b);
            else if constexpr (OP == MX_OP_SUB) return (S)((U)a - (U)b);
            else if constexpr (OP == MX_OP_MUL) return (S)((U)a * (U)b);
            else if constexpr (OP == MX_OP_DIV) {
                if (b == 0) return (S)0;
                if constexpr (Tr::is_signed) {
                    using W = std::conditional_t<(sizeof(S) <= 4), int32_t, int64_t>;
                    W x = a, y = b;
                    if (y == -1) return (S)(0 - (U)x);      // MIN / -1 wraps to MIN
                    return (S)(x / y);
                } else {
                    return (S)((U)a / (U)b);
                }
            } else if constexpr (OP == MX_OP_MAX) return (a < b) ? b : a;
            else if constexpr (OP == MX_OP_MIN) return (b < a) ? b : a;
            else return (S)(a == b ? 1 : 0);
        }
    }
};

}  // namespace mx
