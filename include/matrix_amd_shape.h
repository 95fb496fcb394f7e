/*
 * matrix_amd_shape.h -- host shape helpers that produce the descriptors the kernels consume.
 *
 * C entry points for the broadcast and dim-collapsing helpers of the reference
 * (Matrix.mm:161-331, Mods/Utils.mm:114-435).  They run on the host only, at graph-build
 * time, exactly once per node (Matrix.mm:8312-8331).  Results are written into
 * caller-provided arrays of MX_MAX_DIMS entries; *out_dims receives the collapsed rank.
 * Status codes are mx_status from matrix_amd.h.
 */
#ifndef MATRIX_AMD_SHAPE_H
#define MATRIX_AMD_SHAPE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* collapse_dims with three stride sets (Mods/Utils.mm:169-202): merges axis i into the
 * previous slot when every operand has stride[prev] == stride[i] * shape[i] and the merged
 * extent stays <= size_cap; size-1 axes after axis 0 are dropped. */
int mx_collapse_dims3(const uint32_t* shape, const uint32_t* sA, const uint32_t* sB,
                      const uint32_t* sC, uint32_t dims, uint64_t size_cap,
                      uint32_t* out_shape, uint32_t* out_sA, uint32_t* out_sB,
                      uint32_t* out_sC, uint32_t* out_dims);

/* collapse_dims with two stride sets (Mods/Utils.mm:138-167). */
int mx_collapse_dims2(const uint32_t* shape, const uint32_t* sA, const uint32_t* sB,
                      uint32_t dims, uint64_t size_cap, uint32_t* out_shape,
                      uint32_t* out_sA, uint32_t* out_sB, uint32_t* out_dims);

/* collapse_dims_matmul (Mods/Utils.mm:204-252): batch axes collapse, the last two
 * ([..., M, N]) are copied verbatim. */
int mx_collapse_dims_matmul(const uint32_t* shape, const uint32_t* sA, const uint32_t* sB,
                            const uint32_t* sC, uint32_t dims, uint64_t size_cap,
                            uint32_t* out_shape, uint32_t* out_sA, uint32_t* out_sB,
                            uint32_t* out_sC, uint32_t* out_dims);

/* collapse_dims_reduce with output / input strides and outer_collapsed
 * (Mods/Utils.mm:321-376): the reduced axis is a hard split; with outer_collapsed the output
 * stride index shifts down by one after the axis. */
int mx_collapse_dims_reduce2(const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                             uint32_t dims, int axis, int keep_dims, int outer_collapsed,
                             uint64_t size_cap, uint32_t* out_shape, uint32_t* out_sOut,
                             uint32_t* out_sIn, uint32_t* out_dims);

/* broadcast_shapes (Matrix.mm:161-232): right-aligned NumPy broadcast.  Writes the output
 * shape and contiguous output strides (out_dims = max(d1, d2) entries) and each operand's
 * broadcast shape / strides, 0 on broadcast axes.  MX_ERR_INVALID_ARG on a mismatch. */
int mx_broadcast_shapes(const uint32_t* shape1, const uint32_t* strides1, uint32_t d1,
                        const uint32_t* shape2, const uint32_t* strides2, uint32_t d2,
                        uint32_t* out_shape, uint32_t* out_strides,
                        uint32_t* b1_shape, uint32_t* b1_strides,
                        uint32_t* b2_shape, uint32_t* b2_strides);

/* broadcast_shapes_matmul (Matrix.mm:234-331): operand 1 is [..., M, K], operand 2 is
 * Bt [..., N, K]; batch axes broadcast, output is [..., M, N]. */
int mx_broadcast_shapes_matmul(const uint32_t* shape1, const uint32_t* strides1, uint32_t d1,
                               const uint32_t* shape2, const uint32_t* strides2, uint32_t d2,
                               uint32_t* out_shape, uint32_t* out_strides,
                               uint32_t* b1_shape, uint32_t* b1_strides,
                               uint32_t* b2_shape, uint32_t* b2_strides);

#ifdef __cplusplus
}
#endif
#endif
