/*
 * matrix_amd.h -- C launch ABI of the MI355X (gfx950) evaluation path.
 *
 * This is the boundary between the host graph layer (matrix / Primitive, lazy DFS,
 * compile / execute) and the device.  It replaces the reference's L2 GPU backends and
 * its Metal device manager:
 *   - every call is `extern "C"`, takes plain pointers, sizes and uint32 element strides
 *     (the reference's size_m, Mods/Utils.h:125), and returns an mx_status;
 *   - nothing throws across it; mx_last_error() gives the message of the last failure on
 *     the calling thread;
 *   - launches are asynchronous on the given stream (NULL = the calling thread's stream,
 *     see mx_hip_stream_for_thread); nothing allocates device memory except mx_hip_alloc
 *     (launches take caller workspaces, sized by the *_workspace_bytes queries);
 *   - descriptor arrays (shape / strides) are read on the host during the call and may be
 *     freed as soon as it returns.
 *
 * Element type codes are the reference's dtype codes (matrix.h:35-52).
 */
#ifndef MATRIX_AMD_H
#define MATRIX_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ codes */
typedef enum {
    MX_OK = 0,
    MX_ERR_INVALID_ARG = 1,     /* bad shape / stride / rank / null pointer */
    MX_ERR_UNSUPPORTED = 2,     /* no kernel for this (op, dtype) -- GPUManager.h:64-71 */
    MX_ERR_HIP = 3,             /* a HIP runtime call failed */
    MX_ERR_NOT_INITIALIZED = 4, /* mx_hip_init was not called */
    MX_ERR_WORKSPACE = 5        /* workspace missing or too small */
} mx_status;

/* dtype codes, matrix.h:35-52 */
enum {
    MX_FLOAT32 = 0, MX_FLOAT16 = 1, MX_UINT8 = 2, MX_INT32 = 3, MX_INT16 = 4,
    MX_UINT32 = 5, MX_UINT16 = 6, MX_BOOL = 7, MX_INT8 = 8, MX_COMPLEX64 = 9,
    MX_BFLOAT16 = 10, MX_INT64 = 11, MX_UINT64 = 12
};

/* broadcast binary ops */
enum { MX_OP_ADD = 0, MX_OP_SUB = 1, MX_OP_MUL = 2, MX_OP_DIV = 3,
       MX_OP_MAX = 4, MX_OP_MIN = 5, MX_OP_EQ = 6 };

/* reductions */
enum { MX_RED_SUM = 0, MX_RED_MAX = 1, MX_RED_MIN = 2, MX_RED_ARGMAX = 3, MX_RED_ARGMIN = 4 };

#define MX_MAX_DIMS 8   /* MAX_TENSOR_DIMS, Mods/Utils.h:127 */

const char* mx_last_error(void);
const char* mx_version(void);

/* ------------------------------------------------------------------ device runtime
 * Replaces GlobalGPUManager (Mods/GPUManager.h:26-58, GPUManager.h:1261): device + per-thread
 * stream instead of MTLDevice + thread-local command buffer / encoder. */
int mx_hip_init(int device);
int mx_hip_shutdown(void);
int mx_hip_device_count(int* count);

/* The matrix buffer's MTLBuffer slot (matrix.h:677-680, matrix.h:458-467) becomes a device
 * allocation; the host matrix keeps the atomic refcount. */
int mx_hip_alloc(size_t bytes, void** dptr);
int mx_hip_free(void* dptr);
/* Device allocations (mx_hip_alloc) and frees made so far by this process.  No launch entry point
 * allocates; the counter lets a caller check that a phase such as a graph's execute allocated
 * nothing (the reference's "no buffer is built during EXECUTE", .agents/MemoryManagement.md:335). */
int mx_hip_alloc_stats(uint64_t* allocs, uint64_t* frees);
int mx_hip_h2d(void* dst, const void* src, size_t bytes, void* stream);
int mx_hip_d2h(void* dst, const void* src, size_t bytes, void* stream);
int mx_hip_d2d(void* dst, const void* src, size_t bytes, void* stream);
int mx_hip_memset(void* dst, int value, size_t bytes, void* stream);

/* getCommandBuffer / commitCommandBuffer (GPUManager.h:540-594, GPUManager.h:558-562):
 * one stream per host thread; sync waits and reports any asynchronous kernel error. */
int mx_hip_stream_for_thread(void** stream);
int mx_hip_sync(void* stream);

/* Further streams for independent work (no counterpart in the reference, whose encoder is one
 * in-order queue per thread, GPUManager.h:57-58): a caller that runs independent nodes
 * concurrently creates streams, orders them with events (record on one, wait on another), and
 * destroys them when done.  Streams have the default priority. */
int mx_hip_stream_create(void** stream);
int mx_hip_stream_destroy(void* stream);
int mx_hip_stream_wait_event(void* stream, void* event);

/* Timing (the reference's Timer, Mods/Utils.h:316-335, but on the device clock). */
int mx_hip_event_create(void** event);
int mx_hip_event_destroy(void* event);
int mx_hip_event_record(void* event, void* stream);
int mx_hip_event_elapsed_ms(void* start, void* stop, float* ms);

/* ------------------------------------------------------------------ kernels */

/* R[i] = A[i] op B[i] over a collapsed broadcast iteration space.
 * Replaces add/subtract/multiply/divide_gpu_brodcasted (Matrix.mm:7709-8238), the binary
 * max/min backends (Matrix.mm:13378-13478, Matrix.mm:14668-14783) and equal_backend
 * (Matrix.mm:14469-14540).  The arrays are exactly CollapsedDims_3 (Mods/Utils.h:142-148)
 * from collapse_dims (Mods/Utils.mm:169-202): shape, stridesC (= sR), stridesA, stridesB.
 * cdims == 0 is the rank-0 case (Matrix.mm:7460-7469).  A, B and R share one dtype: any of the
 * 12 real codes for every op; MX_COMPLEX64 for ADD / SUB / MUL / DIV only, as the reference
 * instantiates it (BrodcastedAdd.metal:95 and siblings), else MX_ERR_UNSUPPORTED. */
int mx_launch_bcast_binary(int op, int dtype, int cdims, const uint32_t* shape,
                           const uint32_t* sR, const uint32_t* sA, const uint32_t* sB,
                           void* R, const void* A, const void* B, void* stream);

/* out[g] = reduce_{i < n_reduce} in[offset(g) + i * reduce_stride] for every output g,
 * out written contiguously.  Replaces sum(out, axis, keepdims, dev) (Matrix.mm:15099-15208),
 * max / min (Matrix.mm:14812-15059) and argmax / argmin (Matrix.mm:16182-16458).  The arrays
 * are exactly CollapsedDims_2 from collapse_dims_reduce (Mods/Utils.mm:321-376): shape,
 * stridesA (= sOut), stridesB (= sIn); reduce_stride / n_reduce are strides()[axis] and
 * shape()[axis] (Matrix.mm:15104-15105).  ARGMAX / ARGMIN write int32.  When the reduced axis
 * is split over several blocks (few outputs, long axis), the workspace holds their partials and
 * a second launch combines them; its size comes from mx_reduce_workspace_bytes (0 means none is
 * needed, and then workspace may be NULL).  Launches that share one workspace must not overlap
 * in time (use one stream). */
int mx_reduce_workspace_bytes(int op, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                              int cdims, const uint32_t* shape, const uint32_t* sOut,
                              const uint32_t* sIn, size_t* bytes);
int mx_launch_reduce(int op, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                     int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                     void* out, const void* in, void* workspace, size_t workspace_bytes,
                     void* stream);

/* No counterpart in the reference: mx_launch_reduce for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * takes no workspace: a reduction whose axis is split over blocks keeps its partials in a fixed
 * 4 MiB device array that the library holds on each GPU until the process ends (set up by
 * mx_hip_init for its device).  Reductions needing more than that (mx_reduce_workspace_bytes
 * above 4 MiB) fail with MX_ERR_WORKSPACE.  Outputs equal mx_launch_reduce's bit for bit.  The
 * call allocates nothing.  Every call on one GPU shares that array: calls that overlap in time
 * on one GPU (two streams, two threads) race, so issue them on one stream. */
#define MX_REDUCE_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)
int mx_launch_reduce_noalloc(int op, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                             int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                             void* out, const void* in, void* stream);

/* n (<= MX_REDUCE_GROUP_MAX) reductions of one dtype over one descriptor (the arguments of
 * mx_launch_reduce), member k with its own op ops[k], input ins[k], output outs[k] and workspace
 * workspaces[k] of workspace_bytes[k] bytes (its mx_reduce_workspace_bytes; the two arrays may be
 * NULL when no member needs one).  Each output equals that of mx_launch_reduce(ops[k], ...,
 * outs[k], ins[k], ...) bit for bit.  Float dtypes run as one launch (plus one combine launch for
 * a split axis), the others as one launch per member.  The members must be independent: no
 * output may overlap another output or any input.  No counterpart in the reference, which
 * launches each Sum / Max / Min / ArgMax / ArgMin (Matrix.mm:15099-15208, Matrix.mm:14812-15059,
 * Matrix.mm:16182-16458) on its own: the graph layer's horizontal fusion of independent
 * reductions with the same collapsed descriptor, so that several of them stream through HBM in
 * one launch instead of paying a launch's ramp-up and tail each. */
#define MX_REDUCE_GROUP_MAX 8
int mx_launch_reduce_group(int n, const int* ops, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                           int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                           void* const* outs, const void* const* ins, void* const* workspaces,
                           const size_t* workspace_bytes, void* stream);

/* R = A op B exactly as mx_launch_bcast_binary, and out[r] = red_op over R[r * n .. r * n + n)
 * (the values as stored in R; R must be contiguous, n must divide the result's size and
 * n * sizeof(dtype) <= 16384).  out is contiguous, one element per row (int32 for ARGMAX /
 * ARGMIN, the dtype otherwise); results equal mx_launch_bcast_binary followed by
 * mx_launch_reduce over the rows bit for bit, except that float sums may round differently
 * (another fixed summation order).  No counterpart in the reference: the graph layer's fusion of
 * a broadcast node (add/sub/mul/divide/max/min_gpu_brodcasted, Matrix.mm:7709-8238) with a
 * Sum / Max / Min / ArgMax / ArgMin over its last axis (Matrix.mm:15099-15208,
 * Matrix.mm:14812-15059, Matrix.mm:16182-16458), which writes R and reduces it from registers.
 * Float dtypes with Sum / Max / Min run fused; the rest run the two kernels in turn.
 * MX_ERR_UNSUPPORTED when those rows would need a split reduction's workspace. */
int mx_launch_bcast_binary_reduce_rows(int op, int red_op, int dtype, int cdims, const uint32_t* shape,
                                       const uint32_t* sR, const uint32_t* sA, const uint32_t* sB, uint32_t n,
                                       void* R, const void* A, const void* B, void* out, void* stream);

/* No counterpart in the reference: the gradient that the vjp of Max / Min (MaxPrimitive /
 * MinPrimitive, primitives.cpp:2604-2608) sends to one operand, built there from four nodes:
 * mask_b = equal(b, max(a, b)) (min for MX_OP_MIN), then R = G * (1 - mask_b) for side 0 (a)
 * or R = G * mask_b for side 1 (b), in one launch for a graph's backward pass.  The arrays are
 * the CollapsedDims_3 of R = broadcast(A, B) as for mx_launch_bcast_binary; G is read with R's
 * strides.  float32 / float16 / bfloat16; each element equals the four broadcast launches'
 * result bit for bit. */
int mx_launch_max_grad(int op, int side, int dtype, int cdims, const uint32_t* shape, const uint32_t* sR,
                       const uint32_t* sA, const uint32_t* sB, void* R, const void* A, const void* B,
                       const void* G, void* stream);

/* C[b, m, n] = sum_k A[b, m, k] * Bt[b, n, k].  Replaces dot_gpu / batched_dot_gpu
 * (Matrix.mm:7198-7291).  The arrays are exactly CollapsedDims_3 from collapse_dims_matmul
 * (Mods/Utils.mm:204-252): shapeC = [batch..., M, N], sA / sBt / sC per axis, whose last
 * entry is the K stride of A and of Bt (the reference requires 1 there; any value is
 * accepted here) and the N stride of C.  float32 runs on fp32 MFMA, float16 / bfloat16 on
 * 16-bit MFMA with fp32 accumulation; integer types accumulate in their own type (wrap).
 * This form takes no workspace, so it never splits the K range over blocks (a product with few
 * output tiles then leaves CUs idle); mx_launch_batched_matmul_ws below does. */
int mx_launch_batched_matmul(int dtype, int cdims, const uint32_t* shapeC,
                             const uint32_t* sA, const uint32_t* sBt, const uint32_t* sC,
                             uint32_t K, void* C, const void* A, const void* Bt, void* stream);

/* mx_launch_batched_matmul with a caller workspace, as the reference's primitives allocate
 * during COMPILE and never during EXECUTE (primitives.cpp:454-470): when the output has too few
 * tiles to fill the CUs (or, for at most 16 rows of A with Bt N-major, too few 128-byte column
 * groups), the K range is split over blocks, the fp32 partials go to the
 * workspace and a second launch sums them in split order (deterministic).  The size comes from
 * mx_matmul_workspace_bytes (0: the product never splits, workspace may be NULL); a workspace
 * smaller than that (or NULL) runs the product unsplit.  Results differ from the unsplit form
 * only in the fp32 summation order.  Launches sharing a workspace must not overlap in time. */
int mx_matmul_workspace_bytes(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                              const uint32_t* sBt, const uint32_t* sC, uint32_t K, size_t* bytes);
int mx_launch_batched_matmul_ws(int dtype, int cdims, const uint32_t* shapeC,
                                const uint32_t* sA, const uint32_t* sBt, const uint32_t* sC,
                                uint32_t K, void* C, const void* A, const void* Bt,
                                void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference: a Dot node followed by a broadcast Add of a bias row and a
 * Max / Min against a scalar (DotPrimitive, primitives.cpp:5464-5626; AdditionPrimitive,
 * primitives.cpp:397-560; MaxPrimitive / MinPrimitive, primitives.cpp:2515-2824), the bias +
 * ReLU of a dense layer, in one call for a graph compiler that fuses the three nodes.  Computes
 * C as mx_launch_batched_matmul_ws does (same workspace rules), then Z = C + bias (bias: N
 * contiguous elements, broadcast over the batch and M) and H = max(Z, s) (act_op MX_OP_MAX) or
 * min(Z, s) (MX_OP_MIN), s one element at act_scalar, each element exactly as
 * mx_launch_bcast_binary computes it, so C, Z and H equal those three launches bit for bit.
 * float32 / float16 / bfloat16; C, Z and H contiguous with C's shape.  With a split K range the
 * combine launch writes C, Z and H; else one epilogue launch reads C once and writes Z and H. */
int mx_launch_batched_matmul_bias_act(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                                      const uint32_t* sBt, const uint32_t* sC, uint32_t K, void* C,
                                      const void* A, const void* Bt, const void* bias, void* Z, int act_op,
                                      const void* act_scalar, void* H, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* Channels-last N-D convolution, the argument set of conv_gpu (Matrix.mm:12335-12395) /
 * conv2d_gpu (Matrix.mm:5521-5559): input [N, S1..Sn, C], kernel [O, K1..Kn, C/groups],
 * output [N, O1..On, O], each with arbitrary element strides; pad_lo / stride / dil_rhs
 * (kernel dilation) / dil_lhs (input dilation) have nspatial entries; flip != 0 reads the
 * kernel back to front.  Operands that are not channel-contiguous are packed into the
 * workspace first (size from mx_conv_workspace_bytes). */
int mx_conv_workspace_bytes(int dtype, int nspatial, const uint32_t* in_shape,
                            const uint32_t* k_shape, const uint32_t* out_shape,
                            const uint32_t* in_strides, const uint32_t* k_strides,
                            const uint32_t* out_strides, int groups, size_t* bytes);
int mx_launch_conv_nd(int dtype, int nspatial, const uint32_t* in_shape,
                      const uint32_t* k_shape, const uint32_t* out_shape,
                      const uint32_t* in_strides, const uint32_t* k_strides,
                      const uint32_t* out_strides, const int* pad_lo, const int* stride,
                      const int* dil_rhs, const int* dil_lhs, int groups, int flip,
                      void* out, const void* in, const void* kern,
                      void* workspace, size_t workspace_bytes, void* stream);

/* dst[sum idx * sDst] = cast(src[sum idx * sSrc]) over a collapsed space.  Replaces
 * copyGPUinplace / copyGPUinplaceTypeCasted and the CopyInplaceGPU kernels
 * (Matrix.mm:1699-1976, Copy.metal:14-80).  Any pair of the 12 real codes; within one dtype
 * (MX_COMPLEX64 included) the element's bytes move unchanged; a real code -> MX_COMPLEX64 gives
 * (float(v), 0) (complex.h:22); MX_COMPLEX64 -> a real code is MX_ERR_UNSUPPORTED. */
int mx_launch_copy_strided(int dst_dtype, int src_dtype, int cdims, const uint32_t* shape,
                           const uint32_t* sDst, const uint32_t* sSrc,
                           void* dst, const void* src, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MATRIX_AMD_H */
