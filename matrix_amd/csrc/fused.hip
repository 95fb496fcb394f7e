// fused.hip -- a broadcast binary op whose result is also reduced over its rows.
//
// R = A op B exactly as mx_launch_bcast_binary computes it (elementwise.hpp), and out[r] = Sum /
// Max / Min of R[r * n .. r * n + n) -- the values as stored in R -- with the reduction rules of
// reduce_ops.hpp.  This is the graph layer's fusion of a BrodcastedAdd/Sub/Mul/Divide/Max/Min
// node (Matrix.mm:7411-7707, Matrix.mm:13378-13478) with a Sum / Max / Min over its last axis
// (Matrix.mm:15099-15208, Matrix.mm:14812-15059): R is still written in full (it is a node of the
// graph), but the reduction reads it from registers instead of from HBM, so the pair moves
// |A| + |B| + |R| + |out| bytes instead of |A| + |B| + 2 |R| + |out|.
//
// One wave per row of R: lane l takes the row's 16-byte vectors l, l + 64, ..., four in flight,
// computes them, stores them and steps them into its state in index order; the wave combines
// its lanes' states (index-ordered, so Max / Min keep the first of equal values).  Float sums
// accumulate in fp32 over the stored (rounded) values, as the unfused Sum does, in a different
// but fixed order.  Shapes, ops and dtypes outside this path run the two kernels one after the
// other.
#include "elementwise.hpp"
#include "reduce_ops.hpp"

namespace mx {
namespace {

struct FuseDesc {                   // outer collapsed axes (all but the innermost)
    int n;
    FastDiv shape[MX_MAX_DIMS - 1];
    uint32_t sA[MX_MAX_DIMS - 1], sB[MX_MAX_DIMS - 1];
};

constexpr int kFuseUnroll = 4;

// a_vec / b_vec: the operand's innermost collapsed stride is 1 (else 0: one value per row of the
// innermost axis, repeated across the vector).
template <int DT, int BOP, int ROP>
__global__ __launch_bounds__(256) void bcast_reduce_rows_kernel(typename dt_traits<DT>::S* __restrict__ R,
                                                                const typename dt_traits<DT>::S* __restrict__ A,
                                                                const typename dt_traits<DT>::S* __restrict__ B,
                                                                typename RedSel<DT, ROP>::R::OutT* __restrict__ out,
                                                                uint32_t rows, uint32_t nv, FastDiv inner_vecs,
                                                                FuseDesc fd, int a_vec, int b_vec, int nt) {
    using S = typename dt_traits<DT>::S;
    using Red = typename RedSel<DT, ROP>::R;
    constexpr int VEC = 16 / sizeof(S);
    constexpr int U = kFuseUnroll;
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    struct alignas(16) V { S v[VEC]; };
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t v0 = row * nv;
    typename Red::St st = Red::init();
    for (uint32_t i = lane; i < nv; i += 64 * U) {
        V va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t v = i + 64 * u;
            if (v >= nv) continue;
            const uint32_t g = v0 + v;
            uint32_t orow = inner_vecs.div(g);
            const uint32_t col = (g - orow * inner_vecs.d) * VEC;
            uint64_t oa = 0, ob = 0;
            for (int d = fd.n - 1; d >= 0; --d) {
                const uint32_t q = fd.shape[d].div(orow);
                const uint32_t idx = orow - q * fd.shape[d].d;
                orow = q;
                oa += (uint64_t)idx * fd.sA[d];
                ob += (uint64_t)idx * fd.sB[d];
            }
            if (a_vec) {
                const V* p = reinterpret_cast<const V*>(A + oa + col);
                va[u] = (nt & 1) ? ld_stream(p) : *p;
            }
            else {
                const S x = A[oa];
#pragma unroll
                for (int k = 0; k < VEC; k++) va[u].v[k] = x;
            }
            if (b_vec) {
                const V* p = reinterpret_cast<const V*>(B + ob + col);
                vb[u] = (nt & 2) ? ld_stream(p) : *p;
            }
            else {
                const S x = B[ob];
#pragma unroll
                for (int k = 0; k < VEC; k++) vb[u].v[k] = x;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t v = i + 64 * u;
            if (v >= nv) continue;
            V r;
#pragma unroll
            for (int k = 0; k < VEC; k++) r.v[k] = BinOp<DT, BOP>::apply(va[u].v[k], vb[u].v[k]);
            // a streaming store: the reduction consumes r from registers, and the row written
            // is not read again here (config 1: 7.78-7.90 -> 7.34-7.69 us)
            __builtin_nontemporal_store(__builtin_bit_cast(u4v, r), reinterpret_cast<u4v*>(R + (uint64_t)(v0 + v) * VEC));
#pragma unroll
            for (int k = 0; k < VEC; k++) Red::step(st, r.v[k], v * VEC + k);
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) st = Red::combine(st, Red::shfl(st, m));
    if (lane == 0) out[row] = Red::out(st);
}

// The fast path: float dtypes, Add..Min, Sum / Max / Min, the vector layout of the broadcast
// kernel, R contiguous, rows a whole number of vectors.  Returns false when it does not apply.
template <int DT>
bool launch_fast(int op, int red_op, int cdims, const uint32_t* shape, const uint32_t* sR, const uint32_t* sA,
                 const uint32_t* sB, uint32_t n, uint64_t total, void* R, const void* A, const void* B, void* out,
                 hipStream_t st) {
    using S = typename dt_traits<DT>::S;
    constexpr uint32_t VEC = 16 / sizeof(S);
    if (op > MX_OP_MIN || red_op > MX_RED_MIN || cdims < 1 || n % VEC) return false;
    const int in = cdims - 1;
    if (sR[in] != 1 || sA[in] > 1 || sB[in] > 1 || (sA[in] == 0 && sB[in] == 0) || shape[in] % VEC) return false;
    if ((uintptr_t)R % 16 || (sA[in] == 1 && (uintptr_t)A % 16) || (sB[in] == 1 && (uintptr_t)B % 16)) return false;
    uint64_t want = 1;
    for (int d = in; d >= 0; --d) {                 // R contiguous
        if (shape[d] > 1 && sR[d] != want) return false;
        want *= shape[d];
    }
    FuseDesc fd{};
    fd.n = in;
    for (int d = 0; d < in; d++) {
        if ((sA[in] == 1 && sA[d] % VEC) || (sB[in] == 1 && sB[d] % VEC)) return false;
        fd.shape[d] = FastDiv(shape[d]);
        fd.sA[d] = sA[d];
        fd.sB[d] = sB[d];
    }
    const uint32_t rows = (uint32_t)(total / n);
    const dim3 grid((rows + 3) / 4);
    const FastDiv iv(shape[in] / VEC);
    const int av = sA[in] == 1, bv = sB[in] == 1;
    // an operand that no axis broadcasts is read once: nontemporal loads
    bool sa = av, sb = bv;
    for (int d = 0; d < in; d++) {
        if (shape[d] > 1 && sA[d] == 0) sa = false;
        if (shape[d] > 1 && sB[d] == 0) sb = false;
    }
    const int nt = (sa ? 1 : 0) | (sb ? 2 : 0);
    using OutT = S;
#define MX_FUSE(BOP, ROP) hipLaunchKernelGGL((bcast_reduce_rows_kernel<DT, BOP, ROP>), grid, dim3(256), 0, st, (S*)R, \
                                             (const S*)A, (const S*)B, (OutT*)out, rows, n / VEC, iv, fd, av, bv, nt)
#define MX_FUSE_R(BOP) do { switch (red_op) { case MX_RED_SUM: MX_FUSE(BOP, MX_RED_SUM); break; \
                                              case MX_RED_MAX: MX_FUSE(BOP, MX_RED_MAX); break; \
                                              default: MX_FUSE(BOP, MX_RED_MIN); break; } } while (0)
    switch (op) {
    case MX_OP_ADD: MX_FUSE_R(MX_OP_ADD); break;
    case MX_OP_SUB: MX_FUSE_R(MX_OP_SUB); break;
    case MX_OP_MUL: MX_FUSE_R(MX_OP_MUL); break;
    case MX_OP_DIV: MX_FUSE_R(MX_OP_DIV); break;
    case MX_OP_MAX: MX_FUSE_R(MX_OP_MAX); break;
    default: MX_FUSE_R(MX_OP_MIN); break;
    }
#undef MX_FUSE_R
#undef MX_FUSE
    return true;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_launch_bcast_binary_reduce_rows(int op, int red_op, int dtype, int cdims, const uint32_t* shape,
                                                  const uint32_t* sR, const uint32_t* sA, const uint32_t* sB,
                                                  uint32_t n, void* R, const void* A, const void* B, void* out,
                                                  void* stream) {
    const char* who = "mx_launch_bcast_binary_reduce_rows";
    if (cdims < 0 || cdims > MX_MAX_DIMS) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": cdims outside [0, 8]");
    if (cdims > 0 && (!shape || !sR || !sA || !sB)) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null descriptor");
    if (op < MX_OP_ADD || op > MX_OP_EQ) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": unknown op " + std::to_string(op));
    if (red_op < MX_RED_SUM || red_op > MX_RED_ARGMIN)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": unknown reduction " + std::to_string(red_op));
    uint64_t total = 1;
    for (int d = 0; d < cdims; d++) total *= shape[d];
    if (total == 0) return MX_OK;
    if (n == 0 || total % n) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": row length does not divide the result");
    const size_t es = dtype_size(dtype);
    if (es == 0 || dtype == MX_COMPLEX64) return fail(MX_ERR_UNSUPPORTED, std::string(who) + ": no kernel for dtype " + std::to_string(dtype));
    if ((uint64_t)n * es > 16384) return fail(MX_ERR_UNSUPPORTED, std::string(who) + ": rows above 16 KiB");
    if (total > 0xffffffffull) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": more than 2^32-1 elements");
    if (!R || !A || !B || !out) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null buffer");
    // R must be contiguous for the row reduction
    if (cdims > 0) {
        uint64_t want = 1;
        for (int d = cdims - 1; d >= 0; --d) {
            if (shape[d] > 1 && sR[d] != want)
                return fail(MX_ERR_INVALID_ARG, std::string(who) + ": the result must be contiguous");
            want *= shape[d];
        }
    }
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    bool fast = false;
    if (dtype == MX_FLOAT32) fast = launch_fast<MX_FLOAT32>(op, red_op, cdims, shape, sR, sA, sB, n, total, R, A, B, out, st);
    else if (dtype == MX_FLOAT16) fast = launch_fast<MX_FLOAT16>(op, red_op, cdims, shape, sR, sA, sB, n, total, R, A, B, out, st);
    else if (dtype == MX_BFLOAT16) fast = launch_fast<MX_BFLOAT16>(op, red_op, cdims, shape, sR, sA, sB, n, total, R, A, B, out, st);
    if (fast) {
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    // two launches: the broadcast op, then the rows of R
    const uint32_t rows = (uint32_t)(total / n);
    const uint32_t rshape[1] = {rows}, rso[1] = {1}, rsi[1] = {n};
    size_t ws = 0;
    int rc = mx_reduce_workspace_bytes(red_op, dtype, 1, n, 1, rshape, rso, rsi, &ws);
    if (rc != MX_OK) return rc;
    if (ws) return fail(MX_ERR_UNSUPPORTED, std::string(who) + ": these rows need a split reduction (use the two launches)");
    rc = mx_launch_bcast_binary(op, dtype, cdims, shape, sR, sA, sB, R, A, B, st);
    if (rc != MX_OK) return rc;
    return mx_launch_reduce(red_op, dtype, 1, n, 1, rshape, rso, rsi, out, R, nullptr, 0, st);
}
