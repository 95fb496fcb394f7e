// gemm.hip -- batched C[b, m, n] = sum_k A[b, m, k] * Bt[b, n, k].
//
// Replaces dot_gpu / batched_dot_gpu (Matrix.mm:7198-7291), whose Metal kernel computes one
// output per thread (MatMul.metal:46-102).  The reference always hands the backend A [..., M, K]
// and Bt [..., N, K] with K innermost (dot() packs B^T, Matrix.mm:7074-7089), i.e. both operands
// K-major -- the layout MFMA wants.
//
// float16 / bfloat16 / float32: the matrix-core tile kernel of mfma_tile.hpp (256 x 256 tiles,
//                     256 x 128 when N <= 128).
// Other dtypes:       a scalar kernel accumulating in the element type (wrap-around), as the
//                     reference's `T sum` loop does (Matrix.mm:7187-7191).
// When Bt is shared by the whole batch (batch stride 0) and A / C stack their batches
// contiguously, the batch folds into M.
#include "mfma_tile.hpp"

namespace mx {
namespace {

using tile::GemmArgs;
using tile::MmaTraits;

// Scalar kernel for integer (and bool) dtypes: one output per thread, K loop in the element
// type with wrap-around, any strides.
template <int DT>
__global__ __launch_bounds__(256) void gemm_scalar_kernel(typename dt_traits<DT>::S* __restrict__ C,
                                                          const typename dt_traits<DT>::S* __restrict__ A,
                                                          const typename dt_traits<DT>::S* __restrict__ Bt,
                                                          GemmArgs g) {
    using S = typename dt_traits<DT>::S;
    using U = std::conditional_t<(sizeof(S) <= 4), uint32_t, uint64_t>;
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t per_batch = (uint64_t)g.M * g.N;
    if (t >= per_batch * g.batches) return;
    uint32_t bidx = (uint32_t)(t / per_batch);
    const uint64_t mn = t - (uint64_t)bidx * per_batch;
    const uint32_t m = (uint32_t)(mn / g.N), n = (uint32_t)(mn - (uint64_t)m * g.N);
    uint64_t offA = 0, offB = 0, offC = 0;
    for (int d = g.bd.n - 1; d >= 0; --d) {
        uint32_t q = g.bd.shape[d].div(bidx);
        uint32_t idx = bidx - q * g.bd.shape[d].d;
        bidx = q;
        offA += (uint64_t)idx * g.bd.sA[d];
        offB += (uint64_t)idx * g.bd.sB[d];
        offC += (uint64_t)idx * g.bd.sC[d];
    }
    const S* a = A + offA + (uint64_t)m * g.lda;
    const S* b = Bt + offB + (uint64_t)n * g.ldb;
    if constexpr (DT == MX_BOOL) {
        int acc = 0;               // bool: sum += a * b stored as (sum != 0)
        for (uint32_t k = 0; k < g.K; k++) acc = ((acc + a[(uint64_t)k * g.ka] * b[(uint64_t)k * g.kb]) != 0);
        C[offC + (uint64_t)m * g.ldc + (uint64_t)n * g.cn] = (S)acc;
    } else {
        U acc = 0;
        for (uint32_t k = 0; k < g.K; k++) acc += (U)a[(uint64_t)k * g.ka] * (U)b[(uint64_t)k * g.kb];
        C[offC + (uint64_t)m * g.ldc + (uint64_t)n * g.cn] = (S)acc;
    }
}

template <int DT, int BN>
int launch_mfma_bn(GemmArgs& g, void* C, const void* A, const void* Bt, hipStream_t st) {
    using S = typename MmaTraits<DT>::S;
    constexpr int CE = 16 / sizeof(S);
    // the DMA path addresses a tile's rows with 32-bit byte offsets
    const bool vec = g.ka == 1 && g.kb == 1 && g.lda % CE == 0 && g.ldb % CE == 0 &&
                     (uint64_t)tile::BM * g.lda * sizeof(S) < (1ull << 32) &&
                     (uint64_t)BN * g.ldb * sizeof(S) < (1ull << 32) &&
                     (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 && [&] {
                         for (int d = 0; d < g.bd.n; d++)
                             if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
                         return true;
                     }();
    g.tiles_m = (g.M + tile::BM - 1) / tile::BM;
    g.tiles_n = (g.N + BN - 1) / BN;
    const uint64_t blocks = (uint64_t)g.tiles_m * g.tiles_n * g.batches;
    if (blocks > 0x7fffffffull) return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: grid too large");
    tile::MatrixSrc::Geom geo{};
    if (vec)
        hipLaunchKernelGGL((tile::mfma_tile_kernel<DT, BN, true, tile::MatrixSrc>), dim3((uint32_t)blocks),
                           dim3(tile::NTHREADS), 0, st, (S*)C, (const S*)A, (const S*)Bt, g, geo);
    else
        hipLaunchKernelGGL((tile::mfma_tile_kernel<DT, BN, false, tile::MatrixSrc>), dim3((uint32_t)blocks),
                           dim3(tile::NTHREADS), 0, st, (S*)C, (const S*)A, (const S*)Bt, g, geo);
    MX_HIP(hipGetLastError());
    return MX_OK;
}

template <int DT>
int launch_mfma(GemmArgs& g, void* C, const void* A, const void* Bt, hipStream_t st) {
    return g.N <= 128 ? launch_mfma_bn<DT, 128>(g, C, A, Bt, st) : launch_mfma_bn<DT, 256>(g, C, A, Bt, st);
}

template <int DT>
int launch_scalar(GemmArgs& g, void* C, const void* A, const void* Bt, hipStream_t st) {
    using S = typename dt_traits<DT>::S;
    const uint64_t total = (uint64_t)g.M * g.N * g.batches;
    const uint64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffffull) return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: grid too large");
    hipLaunchKernelGGL((gemm_scalar_kernel<DT>), dim3((uint32_t)blocks), dim3(256), 0, st, (S*)C, (const S*)A,
                       (const S*)Bt, g);
    MX_HIP(hipGetLastError());
    return MX_OK;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_launch_batched_matmul(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                                        const uint32_t* sBt, const uint32_t* sC, uint32_t K, void* C,
                                        const void* A, const void* Bt, void* stream) {
    if (cdims < 2 || cdims > MX_MAX_DIMS)
        return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: cdims " + std::to_string(cdims) + " outside [2, 8]");
    if (!shapeC || !sA || !sBt || !sC) return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: null descriptor");
    GemmArgs g{};
    g.M = shapeC[cdims - 2];
    g.N = shapeC[cdims - 1];
    g.K = K;
    g.lda = sA[cdims - 2];
    g.ka = sA[cdims - 1];
    g.ldb = sBt[cdims - 2];
    g.kb = sBt[cdims - 1];
    g.ldc = sC[cdims - 2];
    g.cn = sC[cdims - 1];
    uint64_t batches = 1;
    for (int d = 0; d < cdims - 2; d++) batches *= shapeC[d];
    if (batches == 0 || g.M == 0 || g.N == 0) return MX_OK;
    if (batches * g.M > 0xffffffffull || batches * g.N > 0xffffffffull)
        return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: extent above 2^32-1 (size_m indexing)");
    if (!C || ((!A || !Bt) && K > 0)) return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: null buffer");
    // Fold the batch into M when Bt is shared by every batch and A and C stack their batches as
    // consecutive row blocks (one batch axis, A stride M*lda, C stride M*ldc).
    g.bd.n = cdims - 2;
    for (int d = 0; d < cdims - 2; d++) {
        g.bd.shape[d] = FastDiv(shapeC[d]);
        g.bd.sA[d] = sA[d]; g.bd.sB[d] = sBt[d]; g.bd.sC[d] = sC[d];
    }
    g.batches = (uint32_t)batches;
    if (cdims == 3 && sBt[0] == 0 && (uint64_t)sA[0] == (uint64_t)g.M * g.lda &&
        (uint64_t)sC[0] == (uint64_t)g.M * g.ldc && batches > 1) {
        g.M = (uint32_t)(batches * g.M);
        g.batches = 1;
        g.bd.n = 0;
    }
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    switch (dtype) {
    case MX_FLOAT32: return launch_mfma<MX_FLOAT32>(g, C, A, Bt, st);
    case MX_FLOAT16: return launch_mfma<MX_FLOAT16>(g, C, A, Bt, st);
    case MX_BFLOAT16: return launch_mfma<MX_BFLOAT16>(g, C, A, Bt, st);
    case MX_INT32: return launch_scalar<MX_INT32>(g, C, A, Bt, st);
    case MX_INT16: return launch_scalar<MX_INT16>(g, C, A, Bt, st);
    case MX_INT8: return launch_scalar<MX_INT8>(g, C, A, Bt, st);
    case MX_INT64: return launch_scalar<MX_INT64>(g, C, A, Bt, st);
    case MX_UINT8: return launch_scalar<MX_UINT8>(g, C, A, Bt, st);
    case MX_UINT16: return launch_scalar<MX_UINT16>(g, C, A, Bt, st);
    case MX_UINT32: return launch_scalar<MX_UINT32>(g, C, A, Bt, st);
    case MX_UINT64: return launch_scalar<MX_UINT64>(g, C, A, Bt, st);
    case MX_BOOL: return launch_scalar<MX_BOOL>(g, C, A, Bt, st);
    default:
        return fail(MX_ERR_UNSUPPORTED, "mx_launch_batched_matmul: no kernel for dtype " + std::to_string(dtype));
    }
}
