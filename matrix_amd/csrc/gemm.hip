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

// Split-K combine: C[b, m, n] = round(sum over s of P[s][b][m][n]), splits in order.
template <int DT>
__global__ __launch_bounds__(256) void splitk_sum_kernel(typename MmaTraits<DT>::S* __restrict__ C,
                                                         const float* __restrict__ P, uint32_t nsplit, GemmArgs g,
                                                         FastDiv fn, FastDiv fm) {
    using S = typename MmaTraits<DT>::S;
    const uint64_t per = (uint64_t)g.batches * g.M * g.N;
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= per) return;
    float acc = P[t];
    for (uint32_t s = 1; s < nsplit; s++) acc += P[(uint64_t)s * per + t];
    const uint32_t tt = (uint32_t)t;                     // the launcher keeps per < 2^32
    uint32_t q = fn.div(tt);
    const uint32_t n = tt - q * g.N;
    uint32_t b = fm.div(q);
    const uint32_t m = q - b * g.M;
    uint64_t offC = 0;
    for (int d = g.bd.n - 1; d >= 0; --d) {
        const uint32_t qq = g.bd.shape[d].div(b);
        offC += (uint64_t)(b - qq * g.bd.shape[d].d) * g.bd.sC[d];
        b = qq;
    }
    S v;
    if constexpr (DT == MX_FLOAT32) v = acc;
    else if constexpr (DT == MX_FLOAT16) v = float_to_half_bits(acc);
    else v = float_to_bf16(acc);
    C[offC + (uint64_t)m * g.ldc + (uint64_t)n * g.cn] = v;
}

// Split-K when the output tiles leave most of the 256 CUs idle: enough K pieces (each at least
// four 128-byte K pairs) to give about two blocks per CU.  Returns 1 for no split.
uint32_t choose_split(const tile::TileShape& ts, const GemmArgs& g, uint32_t pair_elems, uint32_t* ksplit) {
    const uint64_t tiles = (uint64_t)((g.M + ts.bm - 1) / ts.bm) * ((g.N + ts.bn - 1) / ts.bn) * g.batches;
    const uint32_t pairs = g.K / pair_elems;
    if (tiles >= 256 || pairs < 8) return 1;
    uint64_t want = (512 + tiles - 1) / tiles;
    if (want > pairs / 4) want = pairs / 4;
    if (want < 2) return 1;
    const uint32_t pairs_per = (uint32_t)((pairs + want - 1) / want);
    *ksplit = pairs_per * pair_elems;
    return (g.K + *ksplit - 1) / *ksplit;
}

template <int DT>
int launch_mfma(GemmArgs& g, void* C, const void* A, const void* Bt, hipStream_t st) {
    using S = typename MmaTraits<DT>::S;
    constexpr int CE = 16 / sizeof(S);
    const tile::TileShape ts = tile::choose_tile(g.M, g.N, g.batches);
    uint32_t ksplit = 0;
    const uint32_t nsplit = choose_split(ts, g, tile::ROWB / sizeof(S), &ksplit);
    const uint64_t per = (uint64_t)g.batches * g.M * g.N;
    // the DMA path addresses a tile's rows with 32-bit byte offsets
    const bool vec = g.ka == 1 && g.kb == 1 && g.lda % CE == 0 && g.ldb % CE == 0 &&
                     (uint64_t)ts.bm * g.lda * sizeof(S) < (1ull << 32) &&
                     (uint64_t)ts.bn * g.ldb * sizeof(S) < (1ull << 32) &&
                     (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 && [&] {
                         for (int d = 0; d < g.bd.n; d++)
                             if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
                         return true;
                     }();
    const tile::MatrixSrc::Geom geo{};
    const char* who = "mx_launch_batched_matmul";
    if (nsplit > 1 && per < 0xffffffffull) {
        // fp32 partials [split][batch][M][N] in the stream's scratch, then an ordered sum
        void* P = nullptr;
        int rc = stream_scratch(st, (size_t)nsplit * per * sizeof(float), &P);
        if (rc) return rc;
        GemmArgs gp = g;
        gp.ksplit = ksplit;
        gp.ldc = g.N;
        gp.cn = 1;
        rc = vec ? tile::launch_tile_kernel<DT, true, true, tile::MatrixSrc>(ts, gp, geo, P, A, Bt, st, who, nsplit)
                 : tile::launch_tile_kernel<DT, false, true, tile::MatrixSrc>(ts, gp, geo, P, A, Bt, st, who, nsplit);
        if (rc) return rc;
        hipLaunchKernelGGL((splitk_sum_kernel<DT>), dim3((uint32_t)((per + 255) / 256)), dim3(256), 0, st, (S*)C,
                           (const float*)P, nsplit, g, FastDiv(g.N), FastDiv(g.M));
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    if (vec) return tile::launch_tile_kernel<DT, true, false, tile::MatrixSrc>(ts, g, geo, C, A, Bt, st, who);
    return tile::launch_tile_kernel<DT, false, false, tile::MatrixSrc>(ts, g, geo, C, A, Bt, st, who);
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
