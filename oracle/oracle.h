/*
 * oracle.h -- CPU restatement of the reference's CPU eval for the GPU hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (matrix_amd/) never links, loads or falls back to it.
 *
 * Every function restates one CPU backend of the reference, keeping its loop
 * order and per-element arithmetic:
 *   orc_bcast_binary   Matrix.mm:7411-7707 (add/sub/mul/div), Matrix.mm:13378-13478
 *                      (max), Matrix.mm:14668-14783 (min), Matrix.mm:14469-14540 (equal)
 *   orc_reduce         Matrix.mm:15099-15208 (sum), Matrix.mm:14812-14915 (max),
 *                      Matrix.mm:14956-15059 (min), Matrix.mm:16182-16303 (argmax),
 *                      Matrix.mm:16337-16458 (argmin)
 *   orc_batched_matmul Matrix.mm:7108-7196 (dot_cpu / batched_dot_cpu)
 *   orc_conv           Matrix.mm:12397-12500 (conv_cpu) == Matrix.mm:5668-5741 (conv2d_cpu)
 *   orc_copy_strided   matrix.h:1337-1550 (copyCPUinplace / copyCPUinplaceTypeCasted)
 *   complex64          complex.h:18-52 (Add / Sub / Mul / Divide; real -> complex64 casts)
 *
 * Element codes are the reference's dtype codes (matrix.h:35-52).
 * Strides and shapes are element counts in uint32 (Utils.h:125 size_m).
 */
#ifndef MATRIX_AMD_ORACLE_H
#define MATRIX_AMD_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_U8 = 2, ORC_I32 = 3, ORC_I16 = 4, ORC_U32 = 5,
    ORC_U16 = 6, ORC_BOOL = 7, ORC_I8 = 8, ORC_C64 = 9, ORC_BF16 = 10,
    ORC_I64 = 11, ORC_U64 = 12
};
enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3, ORC_MAX = 4, ORC_MIN = 5, ORC_EQ = 6 };
enum { ORC_RSUM = 0, ORC_RMAX = 1, ORC_RMIN = 2, ORC_RARGMAX = 3, ORC_RARGMIN = 4 };
/* Accumulator for sum / matmul / conv on 16-bit floats:
 *   ORC_ACC_LITERAL : the element type itself, rounded after every step, as the reference's
 *                     `T sum` loops do (Matrix.mm:7187, Matrix.mm:5714, Matrix.mm:15201).
 *   ORC_ACC_F32     : one float accumulator, rounded once at the end (same loop order). */
enum { ORC_ACC_LITERAL = 0, ORC_ACC_F32 = 1 };

/* IEEE half / bfloat16 conversions, round-to-nearest-even, NaN payload kept. */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
void orc_f16_to_f32_n(const uint16_t* in, float* out, size_t n);
void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n);
void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n);

/* 0 on success, -1 for an unsupported dtype/op. `total` = number of output elements.
 * cdims == 0 is the rank-0 (scalar op scalar) path. */
int orc_bcast_binary(int op, int dtype, int cdims, const uint32_t* shape,
                     const uint32_t* sR, const uint32_t* sA, const uint32_t* sB,
                     uint64_t total, void* R, const void* A, const void* B);

/* `total_out` output elements written contiguously (out[gid]); the input offset of
 * output gid is decomposed with the collapsed output strides exactly as the reference does. */
int orc_reduce(int op, int dtype, int acc_mode, uint32_t reduce_stride, uint32_t n_reduce,
               int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
               uint64_t total_out, void* out, const void* in, int nthreads);

/* C[b, m, n] = sum_k A[b, m, k] * Bt[b, n, k]; K is contiguous in A and Bt, as the
 * reference's dot() guarantees.  cdims >= 2: shape = [batch..., M, N]. */
int orc_batched_matmul(int dtype, int acc_mode, int cdims, const uint32_t* shape,
                       const uint32_t* sA, const uint32_t* sBt, const uint32_t* sC,
                       uint32_t K, void* C, const void* A, const void* Bt, int nthreads);

/* Channels-last N-D convolution (input [N, S1..Sn, C], kernel [O, K1..Kn, C/groups],
 * output [N, O1..On, O]), arbitrary element strides for all three operands. */
int orc_conv(int dtype, int acc_mode, int nspatial,
             const uint32_t* in_shape, const uint32_t* k_shape, const uint32_t* out_shape,
             const uint32_t* in_strides, const uint32_t* k_strides, const uint32_t* out_strides,
             const int* pad_lo, const int* stride, const int* dil_rhs, const int* dil_lhs,
             int groups, int flip, void* out, const void* in, const void* kern, int nthreads);

/* dst[sum idx*sDst] = cast(src[sum idx*sSrc]) over a collapsed iteration space. */
int orc_copy_strided(int dst_dtype, int src_dtype, int cdims, const uint32_t* shape,
                     const uint32_t* sDst, const uint32_t* sSrc, uint64_t total,
                     void* dst, const void* src);

#ifdef __cplusplus
}
#endif
#endif
