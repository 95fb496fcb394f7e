/*
 * oracle.c -- CPU restatement of the reference's CPU eval (TEST INFRASTRUCTURE ONLY).
 *
 * See oracle.h for the list of reference functions restated here.  Arithmetic follows the
 * reference as compiled for its own platform (clang, arm64):
 *   - 16-bit floats (`float16_t` = __fp16, `bfloat16_t` = __bf16) are storage types: every
 *     op converts to float, computes once, and rounds to nearest-even on store.
 *   - narrow integers promote to int and wrap when stored back (two's complement).
 *   - integer division truncates toward zero; a zero divisor yields 0 and MIN / -1 yields
 *     MIN, which is what arm64 sdiv/udiv return (the reference never guards either case).
 *   - `sum += a * b` in the matmul / conv loops is taken as contracted to one fused
 *     multiply-add, clang's default (-ffp-contract=on) on arm64.
 *   - std::max(a, b) is (a < b) ? b : a and std::min(a, b) is (b < a) ? b : a
 *     (Matrix.mm:13472, Matrix.mm:14777): a NaN in `a` is returned, a NaN in `b` is not.
 * Build with -ffp-contract=off so the compiler adds no contraction of its own.
 */
#include "oracle.h"
#include <math.h>
#include <string.h>
#include <limits.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- 16-bit floats */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));      /* inf / NaN */
    if (exp == 0) {
        if (man == 0) return u2f(sign);                                  /* +-0 */
        /* subnormal: value = man * 2^-24, exact in float */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) {                                           /* inf / NaN */
        if (absu == 0x7f800000u) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | ((absu >> 13) & 0x3ffu));
    }
    int32_t e = (int32_t)(absu >> 23) - 127;                             /* unbiased */
    if (e > 15) return sign | 0x7c00u;                                   /* overflow */
    if (e >= -14) {                                                      /* normal half */
        uint32_t man = absu & 0x7fffffu;
        uint32_t hm = man >> 13, rest = man & 0x1fffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | hm;
        if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) h += 1u;   /* may carry to inf */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return sign;                                            /* rounds to 0 */
    /* subnormal half: value / 2^-24 rounded to an integer, ties to even */
    uint32_t man = (absu & 0x7fffffu) | 0x800000u;                       /* 24-bit significand */
    int shift = -e - 1;                                                  /* e=-15 -> 14 ... e=-25 -> 24 */
    uint32_t q = man >> shift;
    uint32_t rest = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rest > half || (rest == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

void orc_f16_to_f32_n(const uint16_t* in, float* out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]); }
void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]); }
void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n) { for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]); }

/* ---------------------------------------------------------------- element access */
#define LD_F32(x) (x)
#define ST_F32(v) (v)
#define LD_F16(x) orc_f16_to_f32(x)
#define ST_F16(v) orc_f32_to_f16(v)
#define LD_BF16(x) orc_bf16_to_f32(x)
#define ST_BF16(v) orc_f32_to_bf16(v)

/* integer ops in 64-bit two's complement; stores truncate (wrap) */
static inline int64_t idiv_s(int64_t a, int64_t b) {
    if (b == 0) return 0;
    if (a == INT64_MIN && b == -1) return a;
    return a / b;
}
static inline uint64_t idiv_u(uint64_t a, uint64_t b) { return b == 0 ? 0 : a / b; }

/* ---------------------------------------------------------------- broadcast binary */
/* Matmul-free elementwise loop, Matrix.mm:7478-7495: gid decomposed by the collapsed
 * output strides, operands gathered with their own strides, out[gid] written. */
#define BCAST_LOOP(T, OUTT, EXPR)                                                     \
    do {                                                                              \
        const T* pa = (const T*)A; const T* pb = (const T*)B; OUTT* pr = (OUTT*)R;    \
        if (cdims == 0) { T a = pa[0], b = pb[0]; pr[0] = (EXPR); break; }            \
        for (uint64_t gid = 0; gid < total; gid++) {                                  \
            uint64_t ia = 0, ib = 0, rem = gid;                                       \
            for (int i = 0; i < cdims; i++) {                                         \
                uint64_t idx = rem / sR[i];                                           \
                ia += idx * sA[i]; ib += idx * sB[i]; rem %= sR[i];                   \
            }                                                                         \
            T a = pa[ia], b = pb[ib];                                                 \
            pr[gid] = (EXPR);                                                         \
        }                                                                             \
    } while (0)

/* equal_backend, Matrix.mm:14518-14536: gid decomposed by shape from the last axis,
 * written at sum(idx * sR). */
#define EQUAL_LOOP(T, ONE, ZERO, EQ)                                                  \
    do {                                                                              \
        const T* pa = (const T*)A; const T* pb = (const T*)B; T* pr = (T*)R;          \
        int cd = cdims; uint32_t one = 1, zero = 0;                                   \
        const uint32_t* shp = shape; const uint32_t *ssa = sA, *ssb = sB, *ssr = sR;  \
        if (cd == 0) { cd = 1; shp = &one; ssa = &zero; ssb = &zero; ssr = &zero; }   \
        for (uint64_t gid = 0; gid < total; gid++) {                                  \
            uint64_t rem = gid, ia = 0, ib = 0, ir = 0;                               \
            for (int d = cd - 1; d >= 0; --d) {                                       \
                uint64_t idx = rem % shp[d];                                          \
                ia += idx * ssa[d]; ib += idx * ssb[d]; ir += idx * ssr[d];           \
                rem /= shp[d];                                                        \
            }                                                                         \
            T a = pa[ia], b = pb[ib];                                                 \
            pr[ir] = (EQ) ? (ONE) : (ZERO);                                           \
        }                                                                             \
    } while (0)

#define BCAST_FLOATLIKE(T, LD, ST)                                                    \
    switch (op) {                                                                     \
    case ORC_ADD: BCAST_LOOP(T, T, ST(LD(a) + LD(b))); return 0;                      \
    case ORC_SUB: BCAST_LOOP(T, T, ST(LD(a) - LD(b))); return 0;                      \
    case ORC_MUL: BCAST_LOOP(T, T, ST(LD(a) * LD(b))); return 0;                      \
    case ORC_DIV: BCAST_LOOP(T, T, ST(LD(a) / LD(b))); return 0;                      \
    case ORC_MAX: BCAST_LOOP(T, T, (LD(a) < LD(b)) ? b : a); return 0;                \
    case ORC_MIN: BCAST_LOOP(T, T, (LD(b) < LD(a)) ? b : a); return 0;                \
    case ORC_EQ:  EQUAL_LOOP(T, ST(1.0f), ST(0.0f), LD(a) == LD(b)); return 0;        \
    default: return -1;                                                               \
    }

#define BCAST_SIGNED(T)                                                                         \
    switch (op) {                                                                               \
    case ORC_ADD: BCAST_LOOP(T, T, (T)((uint64_t)(int64_t)a + (uint64_t)(int64_t)b)); return 0; \
    case ORC_SUB: BCAST_LOOP(T, T, (T)((uint64_t)(int64_t)a - (uint64_t)(int64_t)b)); return 0; \
    case ORC_MUL: BCAST_LOOP(T, T, (T)((uint64_t)(int64_t)a * (uint64_t)(int64_t)b)); return 0; \
    case ORC_DIV: BCAST_LOOP(T, T, (T)idiv_s((int64_t)a, (int64_t)b)); return 0;               \
    case ORC_MAX: BCAST_LOOP(T, T, (a < b) ? b : a); return 0;                                  \
    case ORC_MIN: BCAST_LOOP(T, T, (b < a) ? b : a); return 0;                                  \
    case ORC_EQ:  EQUAL_LOOP(T, (T)1, (T)0, a == b); return 0;                                  \
    default: return -1;                                                                         \
    }

#define BCAST_UNSIGNED(T)                                                             \
    switch (op) {                                                                     \
    case ORC_ADD: BCAST_LOOP(T, T, (T)((uint64_t)a + (uint64_t)b)); return 0;         \
    case ORC_SUB: BCAST_LOOP(T, T, (T)((uint64_t)a - (uint64_t)b)); return 0;         \
    case ORC_MUL: BCAST_LOOP(T, T, (T)((uint64_t)a * (uint64_t)b)); return 0;         \
    case ORC_DIV: BCAST_LOOP(T, T, (T)idiv_u((uint64_t)a, (uint64_t)b)); return 0;    \
    case ORC_MAX: BCAST_LOOP(T, T, (a < b) ? b : a); return 0;                        \
    case ORC_MIN: BCAST_LOOP(T, T, (b < a) ? b : a); return 0;                        \
    case ORC_EQ:  EQUAL_LOOP(T, (T)1, (T)0, a == b); return 0;                        \
    default: return -1;                                                               \
    }

/* bool operands promote to int; the int result is stored as (result != 0). */
#define BCAST_BOOL()                                                                         \
    switch (op) {                                                                            \
    case ORC_ADD: BCAST_LOOP(uint8_t, uint8_t, (uint8_t)(((int)a + (int)b) != 0)); return 0; \
    case ORC_SUB: BCAST_LOOP(uint8_t, uint8_t, (uint8_t)(((int)a - (int)b) != 0)); return 0; \
    case ORC_MUL: BCAST_LOOP(uint8_t, uint8_t, (uint8_t)(((int)a * (int)b) != 0)); return 0; \
    case ORC_DIV: BCAST_LOOP(uint8_t, uint8_t, (uint8_t)(idiv_s(a, b) != 0)); return 0;      \
    case ORC_MAX: BCAST_LOOP(uint8_t, uint8_t, (a < b) ? b : a); return 0;                   \
    case ORC_MIN: BCAST_LOOP(uint8_t, uint8_t, (b < a) ? b : a); return 0;                   \
    case ORC_EQ:  EQUAL_LOOP(uint8_t, (uint8_t)1, (uint8_t)0, a == b); return 0;             \
    default: return -1;                                                                      \
    }

/* complex64, complex.h:18-52: {re, im} floats.  Multiply is (a, b)c + (-b, a)d
 * (complex.h:36-38); clang's default -ffp-contract=on fuses the first product into the add:
 * re = fma(a, c, -(b d)), im = fma(b, c, a d).  Divide multiplies by conj(rhs) = (c, -d) the same
 * way and divides both parts by mag_sq(rhs) = c c + d d, whose squares are rounded separately
 * (complex.h:40-52).  The reference has complex64 kernels for these four ops only
 * (BrodcastedAdd.metal:95 and siblings). */
typedef struct { float re, im; } orc_c64;
static inline orc_c64 c64_add(orc_c64 x, orc_c64 y) { orc_c64 r = {x.re + y.re, x.im + y.im}; return r; }
static inline orc_c64 c64_sub(orc_c64 x, orc_c64 y) { orc_c64 r = {x.re - y.re, x.im - y.im}; return r; }
static inline orc_c64 c64_mul(orc_c64 x, orc_c64 y) {
    orc_c64 r = {fmaf(x.re, y.re, -(x.im * y.im)), fmaf(x.im, y.re, x.re * y.im)};
    return r;
}
static inline orc_c64 c64_div(orc_c64 x, orc_c64 y) {
    orc_c64 cj = {y.re, -y.im};
    orc_c64 p = c64_mul(x, cj);
    float m = y.re * y.re + y.im * y.im;
    orc_c64 r = {p.re / m, p.im / m};
    return r;
}

#define BCAST_COMPLEX()                                                               \
    switch (op) {                                                                     \
    case ORC_ADD: BCAST_LOOP(orc_c64, orc_c64, c64_add(a, b)); return 0;              \
    case ORC_SUB: BCAST_LOOP(orc_c64, orc_c64, c64_sub(a, b)); return 0;              \
    case ORC_MUL: BCAST_LOOP(orc_c64, orc_c64, c64_mul(a, b)); return 0;              \
    case ORC_DIV: BCAST_LOOP(orc_c64, orc_c64, c64_div(a, b)); return 0;              \
    default: return -1;                                                               \
    }

int orc_bcast_binary(int op, int dtype, int cdims, const uint32_t* shape,
                     const uint32_t* sR, const uint32_t* sA, const uint32_t* sB,
                     uint64_t total, void* R, const void* A, const void* B) {
    switch (dtype) {
    case ORC_C64: BCAST_COMPLEX()
    case ORC_F32: BCAST_FLOATLIKE(float, LD_F32, ST_F32)
    case ORC_F16: BCAST_FLOATLIKE(uint16_t, LD_F16, ST_F16)
    case ORC_BF16: BCAST_FLOATLIKE(uint16_t, LD_BF16, ST_BF16)
    case ORC_I8: BCAST_SIGNED(int8_t)
    case ORC_I16: BCAST_SIGNED(int16_t)
    case ORC_I32: BCAST_SIGNED(int32_t)
    case ORC_I64: BCAST_SIGNED(int64_t)
    case ORC_U8: BCAST_UNSIGNED(uint8_t)
    case ORC_U16: BCAST_UNSIGNED(uint16_t)
    case ORC_U32: BCAST_UNSIGNED(uint32_t)
    case ORC_U64: BCAST_UNSIGNED(uint64_t)
    case ORC_BOOL: BCAST_BOOL()
    default: return -1;
    }
}

/* ---------------------------------------------------------------- reductions */
/* Matrix.mm:15188-15206 and siblings: one sequential pass per output over the reduced
 * axis, input offset from the output index decomposed by the collapsed output strides.
 * cdims == 0 is run as one output with unit strides (Matrix.mm:15133-15138). */
#define RED_PROLOGUE                                                                  \
    uint32_t one = 1;                                                                 \
    const uint32_t *so = sOut, *si = sIn; int cd = cdims;                             \
    if (cd == 0) { cd = 1; so = &one; si = &one; }                                    \
    (void)shape;

#define RED_OFFSET(gid, off)                                                          \
    uint64_t off = 0;                                                                 \
    { uint64_t rem_ = (gid);                                                          \
      for (int i_ = 0; i_ < cd; i_++) { off += (rem_ / so[i_]) * si[i_]; rem_ %= so[i_]; } }

/* Sum with accumulator ACC: ACC_INIT, ACC_ADD(acc, x), ACC_OUT(acc). */
#define SUM_LOOP(T, ACCT, ACC_ADD, ACC_OUT)                                           \
    do {                                                                              \
        const T* pin = (const T*)in; T* po = (T*)out;                                 \
        _Pragma("omp parallel for num_threads(nthreads) schedule(static)")            \
        for (int64_t g = 0; g < (int64_t)total_out; g++) {                            \
            RED_OFFSET((uint64_t)g, off)                                              \
            ACCT acc = 0;                                                             \
            for (uint32_t i = 0; i < n_reduce; i++) {                                 \
                T x = pin[off + (uint64_t)i * reduce_stride];                         \
                acc = ACC_ADD(acc, x);                                                \
            }                                                                         \
            po[g] = ACC_OUT(acc);                                                     \
        }                                                                             \
    } while (0)

/* Max/Min: cur starts at dtype_lowest / dtype_max (matrix.h:271-282) and folds with the
 * std::max / std::min select; the stored value is the selected element's own bits. */
#define EXT_LOOP(T, LD, INIT, BETTER)                                                 \
    do {                                                                              \
        const T* pin = (const T*)in; T* po = (T*)out;                                 \
        _Pragma("omp parallel for num_threads(nthreads) schedule(static)")            \
        for (int64_t g = 0; g < (int64_t)total_out; g++) {                            \
            RED_OFFSET((uint64_t)g, off)                                              \
            T cur = (INIT);                                                           \
            for (uint32_t i = 0; i < n_reduce; i++) {                                 \
                T x = pin[off + (uint64_t)i * reduce_stride];                         \
                if (BETTER(LD(x), LD(cur))) cur = x;                                  \
            }                                                                         \
            po[g] = cur;                                                              \
        }                                                                             \
    } while (0)

/* ArgMax/ArgMin: strict comparison from dtype_lowest / dtype_max, index 0 by default,
 * int32 output (Matrix.mm:16285-16300). */
#define ARG_LOOP(T, LD, INIT, BETTER)                                                 \
    do {                                                                              \
        const T* pin = (const T*)in; int32_t* po = (int32_t*)out;                     \
        _Pragma("omp parallel for num_threads(nthreads) schedule(static)")            \
        for (int64_t g = 0; g < (int64_t)total_out; g++) {                            \
            RED_OFFSET((uint64_t)g, off)                                              \
            T cur = (INIT); int32_t arg = 0;                                          \
            for (uint32_t i = 0; i < n_reduce; i++) {                                 \
                T x = pin[off + (uint64_t)i * reduce_stride];                         \
                if (BETTER(LD(x), LD(cur))) { cur = x; arg = (int32_t)i; }            \
            }                                                                         \
            po[g] = arg;                                                              \
        }                                                                             \
    } while (0)

/* std::max(cur, x) replaces cur iff cur < x; std::min(cur, x) iff x < cur. */
#define GT(x, c) ((c) < (x))
#define LT(x, c) ((x) < (c))

#define F32_ADD(acc, x) ((acc) + (x))
#define IDENT(acc) (acc)
#define F16_LIT_ADD(acc, x) orc_f32_to_f16(orc_f16_to_f32(acc) + orc_f16_to_f32(x))
#define BF16_LIT_ADD(acc, x) orc_f32_to_bf16(orc_bf16_to_f32(acc) + orc_bf16_to_f32(x))
#define F16_F32_ADD(acc, x) ((acc) + orc_f16_to_f32(x))
#define BF16_F32_ADD(acc, x) ((acc) + orc_bf16_to_f32(x))
#define INT_ADD(acc, x) ((acc) + (uint64_t)(int64_t)(x))
#define UINT_ADD(acc, x) ((acc) + (uint64_t)(x))
#define BOOL_ADD(acc, x) ((uint8_t)(((int)(acc) + (int)(x)) != 0))

#define REDUCE_INT(T, TMIN, TMAX, ISSIGNED)                                           \
    switch (op) {                                                                     \
    case ORC_RSUM:                                                                    \
        if (ISSIGNED) SUM_LOOP(T, uint64_t, INT_ADD, (T));                            \
        else SUM_LOOP(T, uint64_t, UINT_ADD, (T));                                    \
        return 0;                                                                     \
    case ORC_RMAX: EXT_LOOP(T, IDENT, (T)(TMIN), GT); return 0;                       \
    case ORC_RMIN: EXT_LOOP(T, IDENT, (T)(TMAX), LT); return 0;                       \
    case ORC_RARGMAX: ARG_LOOP(T, IDENT, (T)(TMIN), GT); return 0;                    \
    case ORC_RARGMIN: ARG_LOOP(T, IDENT, (T)(TMAX), LT); return 0;                    \
    default: return -1;                                                               \
    }

int orc_reduce(int op, int dtype, int acc_mode, uint32_t reduce_stride, uint32_t n_reduce,
               int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
               uint64_t total_out, void* out, const void* in, int nthreads) {
    RED_PROLOGUE
    if (nthreads < 1) nthreads = 1;
    switch (dtype) {
    case ORC_F32:
        switch (op) {
        case ORC_RSUM: SUM_LOOP(float, float, F32_ADD, IDENT); return 0;
        case ORC_RMAX: EXT_LOOP(float, IDENT, -FLT_MAX, GT); return 0;
        case ORC_RMIN: EXT_LOOP(float, IDENT, FLT_MAX, LT); return 0;
        case ORC_RARGMAX: ARG_LOOP(float, IDENT, -FLT_MAX, GT); return 0;
        case ORC_RARGMIN: ARG_LOOP(float, IDENT, FLT_MAX, LT); return 0;
        default: return -1;
        }
    case ORC_F16:
        switch (op) {                         /* lowest/max finite half: +-65504 */
        case ORC_RSUM:
            if (acc_mode == ORC_ACC_LITERAL) SUM_LOOP(uint16_t, uint16_t, F16_LIT_ADD, IDENT);
            else SUM_LOOP(uint16_t, float, F16_F32_ADD, orc_f32_to_f16);
            return 0;
        case ORC_RMAX: EXT_LOOP(uint16_t, LD_F16, (uint16_t)0xfbffu, GT); return 0;
        case ORC_RMIN: EXT_LOOP(uint16_t, LD_F16, (uint16_t)0x7bffu, LT); return 0;
        case ORC_RARGMAX: ARG_LOOP(uint16_t, LD_F16, (uint16_t)0xfbffu, GT); return 0;
        case ORC_RARGMIN: ARG_LOOP(uint16_t, LD_F16, (uint16_t)0x7bffu, LT); return 0;
        default: return -1;
        }
    case ORC_BF16:
        switch (op) {                         /* lowest/max finite bfloat16: +-0x1.fep127 */
        case ORC_RSUM:
            if (acc_mode == ORC_ACC_LITERAL) SUM_LOOP(uint16_t, uint16_t, BF16_LIT_ADD, IDENT);
            else SUM_LOOP(uint16_t, float, BF16_F32_ADD, orc_f32_to_bf16);
            return 0;
        case ORC_RMAX: EXT_LOOP(uint16_t, LD_BF16, (uint16_t)0xff7fu, GT); return 0;
        case ORC_RMIN: EXT_LOOP(uint16_t, LD_BF16, (uint16_t)0x7f7fu, LT); return 0;
        case ORC_RARGMAX: ARG_LOOP(uint16_t, LD_BF16, (uint16_t)0xff7fu, GT); return 0;
        case ORC_RARGMIN: ARG_LOOP(uint16_t, LD_BF16, (uint16_t)0x7f7fu, LT); return 0;
        default: return -1;
        }
    case ORC_I8: REDUCE_INT(int8_t, INT8_MIN, INT8_MAX, 1)
    case ORC_I16: REDUCE_INT(int16_t, INT16_MIN, INT16_MAX, 1)
    case ORC_I32: REDUCE_INT(int32_t, INT32_MIN, INT32_MAX, 1)
    case ORC_I64: REDUCE_INT(int64_t, INT64_MIN, INT64_MAX, 1)
    case ORC_U8: REDUCE_INT(uint8_t, 0, UINT8_MAX, 0)
    case ORC_U16: REDUCE_INT(uint16_t, 0, UINT16_MAX, 0)
    case ORC_U32: REDUCE_INT(uint32_t, 0, UINT32_MAX, 0)
    case ORC_U64: REDUCE_INT(uint64_t, 0, UINT64_MAX, 0)
    case ORC_BOOL:
        switch (op) {
        case ORC_RSUM: SUM_LOOP(uint8_t, uint8_t, BOOL_ADD, IDENT); return 0;
        case ORC_RMAX: EXT_LOOP(uint8_t, IDENT, (uint8_t)0, GT); return 0;
        case ORC_RMIN: EXT_LOOP(uint8_t, IDENT, (uint8_t)1, LT); return 0;
        case ORC_RARGMAX: ARG_LOOP(uint8_t, IDENT, (uint8_t)0, GT); return 0;
        case ORC_RARGMIN: ARG_LOOP(uint8_t, IDENT, (uint8_t)1, LT); return 0;
        default: return -1;
        }
    default: return -1;
    }
}

/* ---------------------------------------------------------------- batched matmul */
/* batched_dot_cpu, Matrix.mm:7139-7196: batch offsets decomposed from the last batch axis,
 * then for (m, n): T sum = 0; for k: sum += A[idxA + k] * Bt[idxB + k].  K is unit-stride in
 * both operands, as dot() packs them before this loop (Matrix.mm:7068-7092): the K strides in
 * sA / sBt are not read, so a strided operand is checked against its packed copy. */
#define MM_LOOP(T, ACCT, STEP, OUT)                                                   \
    do {                                                                              \
        const T* pa = (const T*)A; const T* pb = (const T*)Bt; T* pc = (T*)C;         \
        _Pragma("omp parallel for collapse(2) num_threads(nthreads) schedule(static)")\
        for (int64_t bt = 0; bt < (int64_t)batches; bt++) {                           \
            for (int64_t m = 0; m < (int64_t)M; m++) {                                \
                uint64_t gA = 0, gB = 0, gR = 0, rem = (uint64_t)bt;                  \
                for (int i = cdims - 3; i >= 0; i--) {                                \
                    uint64_t d = rem % shape[i];                                      \
                    gA += d * sA[i]; gB += d * sBt[i]; gR += d * sC[i];               \
                    rem /= shape[i];                                                  \
                }                                                                     \
                for (uint64_t n = 0; n < N; n++) {                                    \
                    uint64_t ia = gA + (uint64_t)m * sA[cdims - 2];                   \
                    uint64_t ib = gB + n * sBt[cdims - 2];                            \
                    uint64_t ir = gR + (uint64_t)m * sC[cdims - 2] + n * sC[cdims - 1];\
                    ACCT acc = 0;                                                     \
                    for (uint32_t k = 0; k < K; k++) {                                \
                        T a = pa[ia + k], b = pb[ib + k];                             \
                        acc = STEP(acc, a, b);                                        \
                    }                                                                 \
                    pc[ir] = OUT(acc);                                                \
                }                                                                     \
            }                                                                         \
        }                                                                             \
    } while (0)

#define F32_FMA(acc, a, b) fmaf((a), (b), (acc))
#define F16_LIT_FMA(acc, a, b) orc_f32_to_f16(fmaf(orc_f16_to_f32(a), orc_f16_to_f32(b), orc_f16_to_f32(acc)))
#define F16_F32_FMA(acc, a, b) fmaf(orc_f16_to_f32(a), orc_f16_to_f32(b), (acc))
#define BF16_LIT_FMA(acc, a, b) orc_f32_to_bf16(fmaf(orc_bf16_to_f32(a), orc_bf16_to_f32(b), orc_bf16_to_f32(acc)))
#define BF16_F32_FMA(acc, a, b) fmaf(orc_bf16_to_f32(a), orc_bf16_to_f32(b), (acc))
#define INT_MAC(acc, a, b) ((acc) + (uint64_t)(int64_t)(a) * (uint64_t)(int64_t)(b))
#define UINT_MAC(acc, a, b) ((acc) + (uint64_t)(a) * (uint64_t)(b))
/* bool: sum + a * b is an int, stored back into the bool accumulator as (value != 0) */
#define BOOL_MAC(acc, a, b) ((uint8_t)(((int)(acc) + (int)(a) * (int)(b)) != 0))

int orc_batched_matmul(int dtype, int acc_mode, int cdims, const uint32_t* shape,
                       const uint32_t* sA, const uint32_t* sBt, const uint32_t* sC,
                       uint32_t K, void* C, const void* A, const void* Bt, int nthreads) {
    if (cdims < 2) return -1;
    if (nthreads < 1) nthreads = 1;
    uint64_t M = shape[cdims - 2], N = shape[cdims - 1], batches = 1;
    for (int i = 0; i < cdims - 2; i++) batches *= shape[i];
    switch (dtype) {
    case ORC_F32: MM_LOOP(float, float, F32_FMA, IDENT); return 0;
    case ORC_F16:
        if (acc_mode == ORC_ACC_LITERAL) MM_LOOP(uint16_t, uint16_t, F16_LIT_FMA, IDENT);
        else MM_LOOP(uint16_t, float, F16_F32_FMA, orc_f32_to_f16);
        return 0;
    case ORC_BF16:
        if (acc_mode == ORC_ACC_LITERAL) MM_LOOP(uint16_t, uint16_t, BF16_LIT_FMA, IDENT);
        else MM_LOOP(uint16_t, float, BF16_F32_FMA, orc_f32_to_bf16);
        return 0;
    case ORC_I8: MM_LOOP(int8_t, uint64_t, INT_MAC, (int8_t)); return 0;
    case ORC_I16: MM_LOOP(int16_t, uint64_t, INT_MAC, (int16_t)); return 0;
    case ORC_I32: MM_LOOP(int32_t, uint64_t, INT_MAC, (int32_t)); return 0;
    case ORC_I64: MM_LOOP(int64_t, uint64_t, INT_MAC, (int64_t)); return 0;
    case ORC_U8: MM_LOOP(uint8_t, uint64_t, UINT_MAC, (uint8_t)); return 0;
    case ORC_U16: MM_LOOP(uint16_t, uint64_t, UINT_MAC, (uint16_t)); return 0;
    case ORC_U32: MM_LOOP(uint32_t, uint64_t, UINT_MAC, (uint32_t)); return 0;
    case ORC_U64: MM_LOOP(uint64_t, uint64_t, UINT_MAC, (uint64_t)); return 0;
    case ORC_BOOL: MM_LOOP(uint8_t, uint8_t, BOOL_MAC, IDENT); return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- convolution */
/* conv_cpu, Matrix.mm:12397-12500.  Per output (n, o_1..o_N, oc): loop over the kernel's
 * (k_1..k_N, c) positions with c fastest; a tap is used iff its sample position
 * o*stride - pad + k*dil (in the input-dilated space) is inside the input and falls on a
 * real (undilated) sample.  conv2d_cpu (Matrix.mm:5668-5741) visits the same taps in the
 * same (kh, kw, c) order. */
#define CONV_LOOP(T, ACCT, STEP, OUT)                                                        \
    do {                                                                                     \
        const T* pin = (const T*)in; const T* pk = (const T*)kern; T* po = (T*)out;          \
        _Pragma("omp parallel for num_threads(nthreads) schedule(static)")                   \
        for (int64_t z = 0; z < (int64_t)outer; z++) {                                       \
            int64_t oidx[8], base[8];                                                        \
            for (uint32_t y = 0; y < out_shape[ns]; y++) {                                   \
                for (int oc = 0; oc < out_c; oc++) {                                         \
                    int g = oc / (out_c / groups);                                           \
                    int c0 = g * cpg;                                                        \
                    int64_t rem = z;                                                         \
                    oidx[ns] = y;                                                            \
                    for (int i = ns - 1; i >= 1; i--) { oidx[i] = rem % out_shape[i]; rem /= out_shape[i]; } \
                    int64_t b = rem;                                                         \
                    for (int i = 1; i <= ns; i++)                                            \
                        base[i] = oidx[i] * stride[i - 1] - pad_lo[i - 1];                   \
                    uint64_t out_off = (uint64_t)b * out_strides[0] + (uint64_t)oc * out_strides[ns + 1]; \
                    for (int i = 1; i <= ns; i++) out_off += (uint64_t)oidx[i] * out_strides[i]; \
                    ACCT acc = 0;                                                            \
                    for (int64_t t = 0; t < kdot; t++) {                                     \
                        int c = (int)(t % cpg);                                              \
                        int64_t rk = t / cpg;                                                \
                        uint64_t ioff = (uint64_t)b * in_strides[0] + (uint64_t)(c0 + c) * in_strides[ns + 1]; \
                        uint64_t koff = (uint64_t)oc * k_strides[0] + (uint64_t)c * k_strides[ns + 1]; \
                        int valid = 1;                                                       \
                        for (int j = ns; j >= 1; j--) {                                      \
                            int64_t kj = rk % k_shape[j];                                    \
                            rk /= k_shape[j];                                                \
                            int64_t s = base[j] + kj * dil_rhs[j - 1];                       \
                            int64_t len = ((int64_t)in_shape[j] - 1) * dil_lhs[j - 1] + 1;   \
                            if (s < 0 || s >= len || (s % dil_lhs[j - 1]) != 0) { valid = 0; break; } \
                            int64_t kr = flip ? ((int64_t)k_shape[j] - 1 - kj) : kj;         \
                            koff += (uint64_t)kr * k_strides[j];                             \
                            ioff += (uint64_t)(s / dil_lhs[j - 1]) * in_strides[j];          \
                        }                                                                    \
                        if (valid) acc = STEP(acc, pk[koff], pin[ioff]);                     \
                    }                                                                        \
                    po[out_off] = OUT(acc);                                                  \
                }                                                                            \
            }                                                                                \
        }                                                                                    \
    } while (0)

int orc_conv(int dtype, int acc_mode, int ns,
             const uint32_t* in_shape, const uint32_t* k_shape, const uint32_t* out_shape,
             const uint32_t* in_strides, const uint32_t* k_strides, const uint32_t* out_strides,
             const int* pad_lo, const int* stride, const int* dil_rhs, const int* dil_lhs,
             int groups, int flip, void* out, const void* in, const void* kern, int nthreads) {
    if (ns < 1 || ns > 6 || groups < 1) return -1;
    if (nthreads < 1) nthreads = 1;
    int out_c = (int)out_shape[ns + 1];
    int cpg = (int)k_shape[ns + 1];
    int64_t kdot = 1;
    for (int i = 1; i <= ns + 1; i++) kdot *= k_shape[i];
    int64_t outer = out_shape[0];
    for (int i = 1; i < ns; i++) outer *= out_shape[i];
    switch (dtype) {
    case ORC_F32: CONV_LOOP(float, float, F32_FMA, IDENT); return 0;
    case ORC_F16:
        if (acc_mode == ORC_ACC_LITERAL) CONV_LOOP(uint16_t, uint16_t, F16_LIT_FMA, IDENT);
        else CONV_LOOP(uint16_t, float, F16_F32_FMA, orc_f32_to_f16);
        return 0;
    case ORC_BF16:
        if (acc_mode == ORC_ACC_LITERAL) CONV_LOOP(uint16_t, uint16_t, BF16_LIT_FMA, IDENT);
        else CONV_LOOP(uint16_t, float, BF16_F32_FMA, orc_f32_to_bf16);
        return 0;
    case ORC_I32: CONV_LOOP(int32_t, uint64_t, INT_MAC, (int32_t)); return 0;
    case ORC_I64: CONV_LOOP(int64_t, uint64_t, INT_MAC, (int64_t)); return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- strided copy + cast */
/* dtype_cast (matrix.h:306-313) is static_cast.  Float -> integer conversions out of the
 * target's range are undefined in C++; this restatement saturates to the 64-bit range and
 * then truncates, which is what arm64's fcvtzs/fcvtzu give, NaN -> 0. */
static inline int64_t f_to_i64(float v) {
    if (v != v) return 0;
    if (v >= 9.2233720368547758e18f) return INT64_MAX;
    if (v <= -9.2233720368547758e18f) return INT64_MIN;
    return (int64_t)v;
}
static inline uint64_t f_to_u64(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 1.8446744073709552e19f) return UINT64_MAX;
    return (uint64_t)v;
}
static inline int32_t f_to_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
static inline uint32_t f_to_u32(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 4294967296.0f) return UINT32_MAX;
    return (uint32_t)v;
}

/* Generic element read into (is_float, f, i, u) and write with cast. */
typedef struct { int kind; float f; int64_t i; uint64_t u; } elem_t;  /* kind 0 float, 1 signed, 2 unsigned */

static elem_t rd(int dt, const void* p, uint64_t off) {
    elem_t e = {0, 0.0f, 0, 0};
    switch (dt) {
    case ORC_F32: e.kind = 0; e.f = ((const float*)p)[off]; break;
    case ORC_F16: e.kind = 0; e.f = orc_f16_to_f32(((const uint16_t*)p)[off]); break;
    case ORC_BF16: e.kind = 0; e.f = orc_bf16_to_f32(((const uint16_t*)p)[off]); break;
    case ORC_I8: e.kind = 1; e.i = ((const int8_t*)p)[off]; break;
    case ORC_I16: e.kind = 1; e.i = ((const int16_t*)p)[off]; break;
    case ORC_I32: e.kind = 1; e.i = ((const int32_t*)p)[off]; break;
    case ORC_I64: e.kind = 1; e.i = ((const int64_t*)p)[off]; break;
    case ORC_U8: e.kind = 2; e.u = ((const uint8_t*)p)[off]; break;
    case ORC_BOOL: e.kind = 2; e.u = ((const uint8_t*)p)[off] != 0; break;
    case ORC_U16: e.kind = 2; e.u = ((const uint16_t*)p)[off]; break;
    case ORC_U32: e.kind = 2; e.u = ((const uint32_t*)p)[off]; break;
    case ORC_U64: e.kind = 2; e.u = ((const uint64_t*)p)[off]; break;
    }
    return e;
}

static void wr(int dt, void* p, uint64_t off, elem_t e) {
    float fv = e.kind == 0 ? e.f : (e.kind == 1 ? (float)e.i : (float)e.u);
    int64_t iv; uint64_t uv;
    if (e.kind == 0) { iv = f_to_i64(e.f); uv = (uint64_t)iv; }
    else if (e.kind == 1) { iv = e.i; uv = (uint64_t)e.i; }
    else { iv = (int64_t)e.u; uv = e.u; }
    switch (dt) {
    case ORC_F32: ((float*)p)[off] = fv; break;
    case ORC_F16: ((uint16_t*)p)[off] = orc_f32_to_f16(fv); break;
    case ORC_BF16: ((uint16_t*)p)[off] = orc_f32_to_bf16(fv); break;
    case ORC_I8: ((int8_t*)p)[off] = (int8_t)(e.kind == 0 ? f_to_i32(e.f) : iv); break;
    case ORC_I16: ((int16_t*)p)[off] = (int16_t)(e.kind == 0 ? f_to_i32(e.f) : iv); break;
    case ORC_I32: ((int32_t*)p)[off] = e.kind == 0 ? f_to_i32(e.f) : (int32_t)iv; break;
    case ORC_I64: ((int64_t*)p)[off] = iv; break;
    case ORC_U8: ((uint8_t*)p)[off] = (uint8_t)(e.kind == 0 ? f_to_u32(e.f) : uv); break;
    case ORC_U16: ((uint16_t*)p)[off] = (uint16_t)(e.kind == 0 ? f_to_u32(e.f) : uv); break;
    case ORC_U32: ((uint32_t*)p)[off] = e.kind == 0 ? f_to_u32(e.f) : (uint32_t)uv; break;
    case ORC_U64: ((uint64_t*)p)[off] = e.kind == 0 ? f_to_u64(e.f) : uv; break;
    case ORC_BOOL: ((uint8_t*)p)[off] = e.kind == 0 ? (e.f != 0.0f) : (uv != 0); break;
    }
}

static size_t orc_size(int dt) {
    switch (dt) {
    case ORC_F32: case ORC_I32: case ORC_U32: return 4;
    case ORC_F16: case ORC_BF16: case ORC_I16: case ORC_U16: return 2;
    case ORC_U8: case ORC_I8: case ORC_BOOL: return 1;
    case ORC_I64: case ORC_U64: case ORC_C64: return 8;
    default: return 0;
    }
}

/* One element of the copy.  Within one dtype the element's bytes move unchanged
 * (static_cast<T>(T), and the reference's blit for contiguous copies, Matrix.mm:1719-1747);
 * a real dtype -> complex64 is complex64(float(v), 0) (complex.h:22), float(v) as for a Float
 * destination; complex64 -> a real dtype has no conversion in the reference's type. */
static void copy_elem(int dst_dtype, int src_dtype, void* dst, uint64_t od, const void* src, uint64_t os) {
    if (dst_dtype == src_dtype) {
        size_t es = orc_size(dst_dtype);
        memcpy((char*)dst + od * es, (const char*)src + os * es, es);
    } else if (dst_dtype == ORC_C64) {
        elem_t e = rd(src_dtype, src, os);
        orc_c64 z = {e.kind == 0 ? e.f : (e.kind == 1 ? (float)e.i : (float)e.u), 0.0f};
        ((orc_c64*)dst)[od] = z;
    } else {
        wr(dst_dtype, dst, od, rd(src_dtype, src, os));
    }
}

int orc_copy_strided(int dst_dtype, int src_dtype, int cdims, const uint32_t* shape,
                     const uint32_t* sDst, const uint32_t* sSrc, uint64_t total,
                     void* dst, const void* src) {
    if (dst_dtype < 0 || src_dtype < 0 || dst_dtype > 12 || src_dtype > 12) return -1;
    if (src_dtype == ORC_C64 && dst_dtype != ORC_C64) return -1;
    if (cdims == 0) { copy_elem(dst_dtype, src_dtype, dst, 0, src, 0); return 0; }
    for (uint64_t gid = 0; gid < total; gid++) {
        uint64_t rem = gid, od = 0, os = 0;
        for (int d = cdims - 1; d >= 0; --d) {
            uint64_t idx = rem % shape[d];
            od += idx * sDst[d]; os += idx * sSrc[d];
            rem /= shape[d];
        }
        copy_elem(dst_dtype, src_dtype, dst, od, src, os);
    }
    return 0;
}
