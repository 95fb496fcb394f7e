// gemm.hip -- batched C[b, m, n] = sum_k A[b, m, k] * Bt[b, n, k].
//
// Replaces dot_gpu / batched_dot_gpu (Matrix.mm:7198-7291), whose Metal kernel computes one
// output per thread (MatMul.metal:46-102).  The reference always hands the backend A [..., M, K]
// and Bt [..., N, K] with K innermost (dot() packs B^T, Matrix.mm:7074-7089), i.e. both operands
// K-major -- the layout MFMA wants.
//
// float16 / bfloat16 / float32: the matrix-core tile kernel of mfma_tile.hpp (256 x 256 tiles,
//                     256 x 128 when N <= 128); at most 16 rows of A (after folding the batch):
//                     a streaming kernel on 16 x 16 MFMAs that reads Bt once.
// Other dtypes:       a scalar kernel accumulating in the element type (wrap-around), as the
//                     reference's `T sum` loop does (Matrix.mm:7187-7191).
// When Bt is shared by the whole batch (batch stride 0) and A / C stack their batches
// contiguously, the batch folds into M.
#include "mfma_tile.hpp"
#include "elementwise.hpp"

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

// Bias + activation epilogue of mx_launch_batched_matmul_bias_act: Z = C + bias[n] and
// H = act(Z, s), elementwise as the broadcast Add and Max / Min kernels compute them, written at
// C's offsets.
struct Epi {
    void* Z;
    void* H;
    const void* bias;       // N elements
    const void* s;          // one element
    int act;                // MX_OP_MAX or MX_OP_MIN
};

template <int DT>
__device__ __forceinline__ void epi_store(const Epi& e, uint64_t off, uint32_t n, typename MmaTraits<DT>::S c) {
    using S = typename MmaTraits<DT>::S;
    const S z = BinOp<DT, MX_OP_ADD>::apply(c, static_cast<const S*>(e.bias)[n]);
    const S sv = *static_cast<const S*>(e.s);
    static_cast<S*>(e.Z)[off] = z;
    static_cast<S*>(e.H)[off] = e.act == MX_OP_MAX ? BinOp<DT, MX_OP_MAX>::apply(z, sv) : BinOp<DT, MX_OP_MIN>::apply(z, sv);
}

// Split-K combine: C[b, m, n] = round(sum over s of P[s][b][m][n]), splits in order (EPI: and the
// bias + activation epilogue from the rounded C).
template <int DT, bool EPI>
__global__ __launch_bounds__(256) void splitk_sum_kernel(typename MmaTraits<DT>::S* __restrict__ C,
                                                         const float* __restrict__ P, uint32_t nsplit, GemmArgs g,
                                                         FastDiv fn, FastDiv fm, Epi e) {
    using S = typename MmaTraits<DT>::S;
    const uint64_t per = (uint64_t)g.batches * g.M * g.N;
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= per) return;
    // splits added in order, 8 loads issued before their adds (a split's partial is otherwise one
    // memory latency each); past the last split the loads repeat it and are not added
    float acc = 0.f;
    for (uint32_t s = 0; s < nsplit; s += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = P[(uint64_t)min(s + j, nsplit - 1) * per + t];
        if (s == 0) acc = v[0];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if ((s > 0 || j > 0) && s + j < nsplit) acc += v[j];
    }
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
    const uint64_t off = offC + (uint64_t)m * g.ldc + (uint64_t)n * g.cn;
    C[off] = v;
    if constexpr (EPI) epi_store<DT>(e, off, n, v);
}

// The epilogue after an unsplit product: C, Z and H contiguous, VEC consecutive elements of one
// row per thread (N % VEC == 0, 16-byte aligned buffers), else one element.
template <int DT, int VEC>
__global__ __launch_bounds__(256) void bias_act_kernel(const typename MmaTraits<DT>::S* __restrict__ C, Epi e,
                                                       uint64_t total, FastDiv fnv) {
    using S = typename MmaTraits<DT>::S;
    struct alignas(VEC * sizeof(S)) Vv { S v[VEC]; };
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (t * VEC >= total) return;
    const uint32_t tv = (uint32_t)t;                      // total / VEC < 2^32 (checked by the launcher)
    const uint32_t n0 = (tv - fnv.div(tv) * fnv.d) * VEC;
    const Vv c = reinterpret_cast<const Vv*>(C)[t];
    const S* bias = static_cast<const S*>(e.bias);
    const S sv = *static_cast<const S*>(e.s);
    Vv z, h;
#pragma unroll
    for (int k = 0; k < VEC; k++) {
        z.v[k] = BinOp<DT, MX_OP_ADD>::apply(c.v[k], bias[n0 + k]);
        h.v[k] = e.act == MX_OP_MAX ? BinOp<DT, MX_OP_MAX>::apply(z.v[k], sv) : BinOp<DT, MX_OP_MIN>::apply(z.v[k], sv);
    }
    reinterpret_cast<Vv*>(e.Z)[t] = z;
    reinterpret_cast<Vv*>(e.H)[t] = h;
}

template <int DT>
int launch_bias_act(const GemmArgs& g, const void* C, const Epi& e, hipStream_t st) {
    using S = typename MmaTraits<DT>::S;
    constexpr int VEC = 16 / sizeof(S);
    const uint64_t total = (uint64_t)g.batches * g.M * g.N;
    const bool vec = g.N % VEC == 0 && (uintptr_t)C % 16 == 0 && (uintptr_t)e.Z % 16 == 0 && (uintptr_t)e.H % 16 == 0;
    if (vec) {
        const uint64_t nt = total / VEC;
        hipLaunchKernelGGL((bias_act_kernel<DT, VEC>), dim3((uint32_t)((nt + 255) / 256)), dim3(256), 0, st, (const S*)C,
                           e, total, FastDiv(g.N / VEC));
    } else {
        hipLaunchKernelGGL((bias_act_kernel<DT, 1>), dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, st, (const S*)C,
                           e, total, FastDiv(g.N));
    }
    MX_HIP(hipGetLastError());
    return MX_OK;
}

// ------------------------------------------------------------------ skinny products (M <= 16)
// A block owns 16 consecutive Bt rows (16 C columns) of one batch; its waves split the K range
// into contiguous pieces.  A step is 64 bytes of K: lane l takes the 16-byte K fragment
// 4 (l / 16) + {0..3} of Bt row (n0 + l % 16) and of A row (l % 16), and a 16 x 16 MFMA takes Bt
// as its row operand and A as its column operand: the result is the C^T tile, lane l holding
// C[l % 16][n0 + 4 (l / 16) + r] in acc[r].  Rows past N or M are clamped to a valid row: they
// only feed result rows / columns that are never stored.  Bt streams from HBM once; A (at most 16
// rows) is re-read from the caches.
//
// Each wave streams its K range in chunks of 512 bytes of each of the block's 16 Bt rows.  A chunk
// is read by 8 load instructions that each cover 512 contiguous bytes of 2 rows (whole lines,
// nontemporal: Bt is read once), written to the wave's own 8 KiB of LDS, and the fragments are
// read back from there.  (Loading the fragments straight from global memory makes every load
// instruction touch 64 bytes of 16 rows; that form streamed 3.66 TB/s on A[8, 4096] x
// Bt[4096, 4096] in f32 against 4.13 here.)  LDS position of 16-byte chunk c of row r: r * 32 + (c ^ r), so
// the 16 rows of one fragment read fall in distinct banks.  For 16-bit data a chunk's A fragments
// (L2 hits) are loaded together with its Bt rows, one chunk ahead, into two register buffers (the
// loop runs two chunks per turn), so no L2 round trip is waited for between chunks (A[8, 4096] x
// Bt[4096, 4096] f16: 9.2 -> 8.4 us).  fp32 loads a chunk's A fragments after staging its Bt rows
// and before the next chunk's Bt loads (A one chunk ahead measured 16.6 -> 17.4 us there).  Per
// wave: two accumulators alternating by step, summed at the end, then the waves' tiles are summed
// in wave order through LDS (deterministic).

typedef float f4v __attribute__((ext_vector_type(4)));

template <int DT> struct SkinnyFrag;
template <> struct SkinnyFrag<MX_FLOAT32> { using V = f4v; };
template <> struct SkinnyFrag<MX_FLOAT16> { using V = tile::h8v; };
template <> struct SkinnyFrag<MX_BFLOAT16> { using V = tile::b8v; };

// Waves per block (measured on A[8|16, K] x Bt[4096|8192, K], K = 4096 | 8192, for 4, 8 and 16
// waves and 512- and 1024-byte chunks: 512-byte chunks; 8 waves for fp32, 4 for 16-bit data,
// whose waves then stream four chunks each instead of two; rotating the waves' K ranges from
// block to block changed nothing; two chunks of Bt ahead instead of one was slower).
template <int DT> constexpr int kSkinnyWaves = DT == MX_FLOAT32 ? 8 : 4;

template <int DT>
__device__ __forceinline__ f4v skinny_mma(typename SkinnyFrag<DT>::V b, typename SkinnyFrag<DT>::V a, f4v acc) {
    if constexpr (DT == MX_FLOAT32) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(b[0], a[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(b[1], a[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(b[2], a[2], acc, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x4f32(b[3], a[3], acc, 0, 0, 0);
    } else if constexpr (DT == MX_FLOAT16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a, acc, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a, acc, 0, 0, 0);
    }
}

// The skinny path applies to 16-bit and fp32 data with unit K strides, 16-byte aligned rows and
// K a whole number of fragments, at most 16 rows of A, and enough column tiles to fill the CUs.
template <int DT>
bool skinny_ok(const GemmArgs& g, const void* A, const void* Bt) {
    using S = typename MmaTraits<DT>::S;
    constexpr uint32_t CE = 16 / sizeof(S);
    if (g.M > 16 || g.ka != 1 || g.kb != 1 || g.K % CE || g.lda % CE || g.ldb % CE) return false;
    if ((uintptr_t)A % 16 || (uintptr_t)Bt % 16 || g.batches > 65535) return false;
    for (int d = 0; d < g.bd.n; d++)
        if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
    return (uint64_t)((g.N + 15) / 16) * g.batches >= 128;
}

// kw: K elements per wave (a multiple of one step).  CVEC: C columns are unit-stride and every
// 4-column group starts 4-element aligned, so a lane's 4 results go out in one store.
template <int DT, bool CVEC>
__global__ __launch_bounds__(64 * kSkinnyWaves<DT>) void gemm_skinny_kernel(
    typename MmaTraits<DT>::S* __restrict__ C, const typename MmaTraits<DT>::S* __restrict__ A,
    const typename MmaTraits<DT>::S* __restrict__ Bt, GemmArgs g, uint32_t kw) {
    using S = typename MmaTraits<DT>::S;
    using V = typename SkinnyFrag<DT>::V;
    constexpr uint32_t CE = 16 / sizeof(S);      // elements per fragment
    constexpr uint32_t KS = 4 * CE;               // K per step (64 bytes of a row)
    constexpr uint32_t CH = 8;                    // steps per chunk (512 bytes of a row)
    constexpr uint32_t KC = CH * KS;
    constexpr uint32_t CPR = CH * 4;              // 16-byte pieces per row of a chunk
    constexpr uint32_t RPI = 64 / CPR;            // rows per load instruction
    constexpr uint32_t NL = 16 / RPI;             // load instructions per chunk
    constexpr int W = kSkinnyWaves<DT>;
    __shared__ V stage[W][16 * CPR];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t i = lane & 15, grp = lane >> 4;
    const uint32_t n0 = blockIdx.x * 16;
    uint32_t b = blockIdx.y;
    uint64_t offA = 0, offB = 0, offC = 0;
    for (int d = g.bd.n - 1; d >= 0; --d) {
        const uint32_t q = g.bd.shape[d].div(b);
        const uint32_t idx = b - q * g.bd.shape[d].d;
        b = q;
        offA += (uint64_t)idx * g.bd.sA[d];
        offB += (uint64_t)idx * g.bd.sB[d];
        offC += (uint64_t)idx * g.bd.sC[d];
    }
    const uint32_t kbeg = min(g.K, wave * kw);
    const uint32_t kend = min(g.K, kbeg + kw);
    const uint32_t lr = lane / CPR, lq = lane % CPR;
    const S* bbase = Bt + offB;
    uint64_t lrow[NL];
#pragma unroll
    for (int j = 0; j < (int)NL; j++) lrow[j] = (uint64_t)min(n0 + RPI * j + lr, g.N - 1) * g.ldb;
    const S* arow = A + offA + (uint64_t)min(i, g.M - 1) * g.lda;
    V* st = stage[wave];
    const V zero = {};
    V R[NL], fa[2][CH];
    f4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
    // Every load is unconditional: an element at or beyond kend is read from element kbeg of the
    // same row instead (in bounds) and replaced by zero where it is used, so no branch separates
    // the loads and each wait names exactly the loads it needs.
    auto load_chunk = [&](uint32_t kc) __attribute__((always_inline)) {
        const uint32_t e = kc + lq * CE;
        const uint32_t ee = e < kend ? e : kbeg;
#pragma unroll
        for (int j = 0; j < (int)NL; j++) R[j] = ld_stream(reinterpret_cast<const V*>(bbase + lrow[j] + ee));
    };
    auto load_a = [&](uint32_t kc, V (&f)[CH]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < (int)CH; s++) {
            const uint32_t k = kc + s * KS + grp * CE;
            f[s] = *reinterpret_cast<const V*>(arow + (k < kend ? k : kbeg));
        }
    };
    auto stage_b = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < (int)NL; j++) {
            const uint32_t r = RPI * j + lr;
            st[r * CPR + (lq ^ r)] = R[j];
        }
    };
    auto compute = [&](uint32_t kc, const V (&f)[CH]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < (int)CH; s++) {
            const bool ok = kc + s * KS + grp * CE < kend;
            const V fb = st[i * CPR + ((s * 4 + grp) ^ i)];
            if (s & 1) acc1 = skinny_mma<DT>(ok ? fb : zero, ok ? f[s] : zero, acc1);
            else acc0 = skinny_mma<DT>(ok ? fb : zero, ok ? f[s] : zero, acc0);
        }
    };
    const uint32_t nch = kend > kbeg ? (kend - kbeg + KC - 1) / KC : 0;
    if constexpr (DT == MX_FLOAT32) {
        // per chunk: stage its Bt rows and load its A fragments, the next chunk's Bt loads, the MFMAs
        if (nch > 0) load_chunk(kbeg);
        for (uint32_t c = 0; c < nch; c++) {
            const uint32_t kc = kbeg + c * KC;
            stage_b();
            load_a(kc, fa[0]);
            __builtin_amdgcn_sched_barrier(0);
            if (c + 1 < nch) load_chunk(kc + KC);
            __builtin_amdgcn_sched_barrier(0);
            compute(kc, fa[0]);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        // two chunks per turn (fa[0] holds even chunks' A, fa[1] odd ones'); per chunk: stage its Bt
        // rows, the next chunk's Bt and A loads, the MFMAs.  Staging overwrites LDS this wave read
        // for the last chunk (a wave's LDS accesses are in order).
        if (nch > 0) {
            load_chunk(kbeg);
            load_a(kbeg, fa[0]);
        }
        uint32_t c = 0;
        for (; c + 2 <= nch; c += 2) {
            const uint32_t kc = kbeg + c * KC;
            stage_b();
            __builtin_amdgcn_sched_barrier(0);
            load_chunk(kc + KC);
            load_a(kc + KC, fa[1]);
            __builtin_amdgcn_sched_barrier(0);
            compute(kc, fa[0]);
            __builtin_amdgcn_sched_barrier(0);
            stage_b();
            __builtin_amdgcn_sched_barrier(0);
            if (c + 2 < nch) {
                load_chunk(kc + 2 * KC);
                load_a(kc + 2 * KC, fa[0]);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(kc + KC, fa[1]);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < nch) {
            stage_b();
            compute(kbeg + c * KC, fa[0]);
        }
    }
    f4v acc = acc0 + acc1;
    __shared__ f4v part[W - 1][64];
    if (wave > 0) part[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; w++) acc += part[w][lane];
    if (i >= g.M) return;
    const uint32_t nb = n0 + 4 * grp;
    S* crow = C + offC + (uint64_t)i * g.ldc;
    S o[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        if constexpr (DT == MX_FLOAT32) o[r] = acc[r];
        else if constexpr (DT == MX_FLOAT16) o[r] = float_to_half_bits(acc[r]);
        else o[r] = float_to_bf16(acc[r]);
    }
    if constexpr (CVEC) {
        if (nb < g.N) {
            struct alignas(4 * sizeof(S)) Q { S v[4]; } q{{o[0], o[1], o[2], o[3]}};
            *reinterpret_cast<Q*>(crow + nb) = q;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (nb + r < g.N) crow[(uint64_t)(nb + r) * g.cn] = o[r];
    }
}

template <int DT>
int launch_skinny(const GemmArgs& g, void* C, const void* A, const void* Bt, hipStream_t st) {
    using S = typename MmaTraits<DT>::S;
    constexpr uint32_t KS = 4 * (16 / sizeof(S));
    constexpr int W = kSkinnyWaves<DT>;
    uint32_t kw = (g.K + W - 1) / W;
    kw = (kw + KS - 1) / KS * KS;
    bool cvec = g.cn == 1 && g.N % 4 == 0 && g.ldc % 4 == 0 && (uintptr_t)C % (4 * sizeof(S)) == 0;
    for (int d = 0; cvec && d < g.bd.n; d++)
        if (g.bd.sC[d] % 4) cvec = false;
    const dim3 grid((g.N + 15) / 16, g.batches);
    if (cvec)
        hipLaunchKernelGGL((gemm_skinny_kernel<DT, true>), grid, dim3(64 * W), 0, st, (S*)C, (const S*)A,
                           (const S*)Bt, g, kw);
    else
        hipLaunchKernelGGL((gemm_skinny_kernel<DT, false>), grid, dim3(64 * W), 0, st, (S*)C, (const S*)A,
                           (const S*)Bt, g, kw);
    MX_HIP(hipGetLastError());
    return MX_OK;
}

// ------------------------------------------------------------------ skinny products, B N-major
// C[M <= 16, N] = A[M, K] . B[K, N] with B N-major (Bt's N stride 1: dot()'s B as stored, with no
// transposed copy).  A block owns one 128-byte line of each K row -- NC columns, 64 of a 16-bit
// type or 32 fp32 -- over a range of K: blocks of 16 columns, reading 32- or 64-byte pieces of
// each row, stream at well under half the rate of whole lines (16-bit 4096 x 4096 read by 256
// blocks: 16 us against 7 us).  Few column groups cannot fill the CUs, so K is split over nsplit
// blocks as well, each writing fp32 partials [split][batch][M][N] that splitk_sum_kernel adds in
// order (nsplit 1: C directly).  A block's W waves take consecutive K ranges and add their
// results in wave order.
//
// Per wave, a chunk of KC = 64 K rows x 128 bytes is staged in LDS (8 loads of 8 rows per lane).
// Fragments: 16-bit through two transposing LDS reads per 16-column tile (ds_read_b64_tr_b16:
// within a 16-lane group, lanes 4e .. 4e + 3 address K row e of a 4 x 16 block, 8 bytes each, and
// lane j receives column j); fp32 through four 4-byte reads.
template <int DT> struct SkinnyNN {
    using S = typename MmaTraits<DT>::S;
    static constexpr uint32_t CE = 16 / sizeof(S);       // elements per 16-byte piece
    static constexpr uint32_t NC = 128 / sizeof(S);      // columns per block
    static constexpr uint32_t NT = NC / 16;              // 16-column MFMA tiles
    static constexpr uint32_t KS = 4 * CE;               // K per MFMA step
    static constexpr uint32_t KC = 64;                   // K rows per chunk
    static constexpr int W = 8;                          // waves per block
};

// Blocks the split aims for (column groups x batches x splits).
constexpr uint64_t kSkinnyNNBlocks = 256;

// Byte c of staged K row r.  16-bit: a half-wave's transposing read takes one 32-byte column
// segment of K rows b .. b + 3 and b + 8 .. b + 11 (b a multiple of 4); segment c / 32 of row r
// sits at c / 32 ^ (bit 1 of r | bit 3 of r << 1), which gives those 8 rows 8 distinct 32-byte
// bank groups.  fp32: a read takes 64 bytes of K rows r, r + 4, r + 8, r + 12; rows swap within
// pairs on bit 2 of r (alternating row parity) and the 64-byte halves swap on bit 3, four
// distinct 64-byte bank quarters.
template <int DT>
__device__ __forceinline__ uint32_t skinny_nn_off(uint32_t r, uint32_t c) {
    if constexpr (DT == MX_FLOAT32)
        return (r ^ ((r >> 2) & 1)) * 128 + (c ^ (((r >> 3) & 1) << 6));
    else
        return r * 128 + (c ^ ((((r >> 1) & 1) | ((r >> 2) & 2)) << 5));
}

// The N-major skinny path: at most 16 rows of A (unit K stride), B N-major, 16-byte pieces.
template <int DT>
bool skinny_nn_ok(const GemmArgs& g, const void* A, const void* Bt) {
    constexpr uint32_t CE = SkinnyNN<DT>::CE;
    if (g.M > 16 || g.ka != 1 || g.ldb != 1 || g.K % CE || g.lda % CE || g.kb % CE || g.N % CE) return false;
    if ((uintptr_t)A % 16 || (uintptr_t)Bt % 16 || g.batches > 65535) return false;
    for (int d = 0; d < g.bd.n; d++)
        if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
    return true;
}

// K splits: enough for kSkinnyNNBlocks blocks, at most one per chunk of every wave.
template <int DT>
uint32_t skinny_nn_splits(const GemmArgs& g) {
    using P = SkinnyNN<DT>;
    const uint64_t blocks = (uint64_t)((g.N + P::NC - 1) / P::NC) * g.batches;
    if (blocks >= kSkinnyNNBlocks) return 1;
    uint64_t want = (kSkinnyNNBlocks + blocks - 1) / blocks;
    const uint64_t most = g.K / (P::W * P::KC);
    if (want > most) want = most;
    return want < 1 ? 1 : (uint32_t)want;
}

// kw: K elements per wave (a multiple of one step); wave w of split sp takes K from
// (sp W + w) kw.  SPLIT: Cv is the fp32 partials, else C.
template <int DT, bool SPLIT>
__global__ __launch_bounds__(64 * SkinnyNN<DT>::W) void gemm_skinny_nn_kernel(
    void* __restrict__ Cv, const typename MmaTraits<DT>::S* __restrict__ A,
    const typename MmaTraits<DT>::S* __restrict__ Bt, GemmArgs g, uint32_t ncg, uint32_t kw) {
    using P = SkinnyNN<DT>;
    using S = typename P::S;
    using V = typename SkinnyFrag<DT>::V;
    constexpr uint32_t CE = P::CE, NC = P::NC, NT = P::NT, KS = P::KS, KC = P::KC;
    constexpr uint32_t SPC = KC / KS;              // MFMA steps per chunk
    constexpr int W = P::W;
    __shared__ __align__(16) char stage[W][KC * 128];
    __shared__ f4v part[W - 1][NT][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t i = lane & 15, grp = lane >> 4;
    const uint32_t cg = blockIdx.x % ncg, sp = blockIdx.x / ncg;
    const uint32_t n0 = cg * NC;
    uint32_t b = blockIdx.y;
    uint64_t offA = 0, offB = 0, offC = 0;
    for (int d = g.bd.n - 1; d >= 0; --d) {
        const uint32_t q = g.bd.shape[d].div(b);
        const uint32_t idx = b - q * g.bd.shape[d].d;
        b = q;
        offA += (uint64_t)idx * g.bd.sA[d];
        offB += (uint64_t)idx * g.bd.sB[d];
        offC += (uint64_t)idx * g.bd.sC[d];
    }
    const uint32_t kbeg = (uint32_t)min((uint64_t)g.K, ((uint64_t)sp * W + wave) * kw);
    const uint32_t kend = min(g.K, kbeg + kw);
    const uint32_t lr = lane >> 3, lp = lane & 7;      // K row within a load instruction, 16-byte piece
    uint32_t pc = n0 + lp * CE;
    if (pc >= g.N) pc = n0;                            // pieces past N re-read the group's first (never stored)
    const S* bcol = Bt + offB + pc;
    const S* arow = A + offA + (uint64_t)min(i, g.M - 1) * g.lda;
    char* stb = stage[wave];
    const V zero = {};
    V R[8], fa[SPC];
    f4v acc[NT];
#pragma unroll
    for (int t = 0; t < (int)NT; t++) acc[t] = f4v{0.f, 0.f, 0.f, 0.f};
    // Every load is unconditional: a K row at or beyond kend is read from K row kbeg instead (in
    // bounds) and replaced by zero where it is used.
    auto load_chunk = [&](uint32_t kc) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t k = kc + 8 * j + lr;
            R[j] = ld_stream(reinterpret_cast<const V*>(bcol + (uint64_t)(k < kend ? k : kbeg) * g.kb));
        }
    };
    auto load_a = [&](uint32_t kc) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < (int)SPC; s++) {
            const uint32_t k = kc + s * KS + grp * CE;
            fa[s] = *reinterpret_cast<const V*>(arow + (k < kend ? k : kbeg));
        }
    };
    auto stage_b = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; j++) *reinterpret_cast<V*>(stb + skinny_nn_off<DT>(8 * j + lr, lp * 16)) = R[j];
    };
    // lane (i, grp)'s fragment of step s, tile t: column n0 + 16 t + i, K rows s KS + grp CE .. + CE - 1
    auto read_b = [&](uint32_t s, uint32_t t) __attribute__((always_inline)) -> V {
        if constexpr (DT == MX_FLOAT32) {
            V v;
#pragma unroll
            for (int j = 0; j < 4; j++)
                v[j] = *reinterpret_cast<const float*>(stb + skinny_nn_off<DT>(s * KS + grp * CE + j, t * 64 + i * 4));
            return v;
        } else {
            const uint32_t r = s * KS + grp * CE + (i >> 2), c = t * 32 + (lane & 3) * 8;
            const tile::s4v lo = tile::ds_read_tr16(stb + skinny_nn_off<DT>(r, c));
            const tile::s4v hi = tile::ds_read_tr16(stb + skinny_nn_off<DT>(r + 4, c));
            const auto v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            V out;
            __builtin_memcpy(&out, &v, 16);
            return out;
        }
    };
    auto compute = [&](uint32_t kc) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < (int)SPC; s++) {
            const bool ok = kc + s * KS + grp * CE < kend;
            const V a = ok ? fa[s] : zero;
#pragma unroll
            for (int t = 0; t < (int)NT; t++) {
                const V fb = read_b(s, t);
                acc[t] = skinny_mma<DT>(ok ? fb : zero, a, acc[t]);
            }
        }
    };
    // per chunk: stage its B rows and load its A fragments, the next chunk's B loads, the MFMAs.
    // Staging overwrites LDS this wave read for the last chunk (a wave's LDS accesses are in order).
    const uint32_t nch = kend > kbeg ? (kend - kbeg + KC - 1) / KC : 0;
    if (nch > 0) load_chunk(kbeg);
    for (uint32_t c = 0; c < nch; c++) {
        const uint32_t kc = kbeg + c * KC;
        stage_b();
        load_a(kc);
        __builtin_amdgcn_sched_barrier(0);
        if (c + 1 < nch) load_chunk(kc + KC);
        __builtin_amdgcn_sched_barrier(0);
        compute(kc);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < (int)NT; t++) part[wave - 1][t][lane] = acc[t];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; w++) {
#pragma unroll
        for (int t = 0; t < (int)NT; t++) acc[t] += part[w][t][lane];
    }
    if (i >= g.M) return;
    // lane (i, grp) holds C[i][n0 + 16 t + 4 grp + r] in acc[t][r]; N is a multiple of 4
    if constexpr (SPLIT) {
        const uint64_t per = (uint64_t)g.batches * g.M * g.N;
        float* prow = reinterpret_cast<float*>(Cv) + sp * per + ((uint64_t)blockIdx.y * g.M + i) * g.N;
#pragma unroll
        for (int t = 0; t < (int)NT; t++) {
            const uint32_t n = n0 + 16 * t + 4 * grp;
            if (n < g.N) *reinterpret_cast<f4v*>(prow + n) = acc[t];
        }
    } else {
        S* crow = reinterpret_cast<S*>(Cv) + offC + (uint64_t)i * g.ldc;
#pragma unroll
        for (int t = 0; t < (int)NT; t++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t n = n0 + 16 * t + 4 * grp + r;
                if (n >= g.N) continue;
                S o;
                if constexpr (DT == MX_FLOAT32) o = acc[t][r];
                else if constexpr (DT == MX_FLOAT16) o = float_to_half_bits(acc[t][r]);
                else o = float_to_bf16(acc[t][r]);
                crow[(uint64_t)n * g.cn] = o;
            }
        }
    }
}

// The tile shape of a product: tile::choose_tile's, except that an fp32 A given M-major (unit M
// stride, the vjp's g^T) takes 128 x 128 tiles where that would choose 256 x 256, whose M-major
// fragments spill 48-64 registers (config 5's dW2 = h1^T g2, 4096 x 4096 x 512: the step 0.634-0.643
// -> 0.619-0.626 ms; 256 x 128 tiles no faster).
template <int DT>
tile::TileShape tile_for(const GemmArgs& g) {
    tile::TileShape ts = tile::choose_tile(g.M, g.N, g.batches);
    if (DT == MX_FLOAT32 && g.lda == 1 && g.ka != 1 && ts.bm == 256 && ts.bn == 256) ts = tile::TileShape{128, 128};
    return ts;
}

// Split-K when the output tiles leave most of the 256 CUs idle: enough K pieces (each at least
// four 128-byte K pairs) to give about one block per CU (512 x 4096 x 1024: fp32 86-87 / f16 209
// TFLOP/s, against 75 / 172 at two blocks per CU).  Returns 1 for no split.
uint32_t choose_split(const tile::TileShape& ts, const GemmArgs& g, uint32_t pair_elems, uint32_t* ksplit) {
    const uint64_t tiles = (uint64_t)((g.M + ts.bm - 1) / ts.bm) * ((g.N + ts.bn - 1) / ts.bn) * g.batches;
    const uint32_t pairs = g.K / pair_elems;
    if (tiles >= 256 || pairs < 8) return 1;
    uint64_t want = (256 + tiles - 1) / tiles;
    if (want > pairs / 4) want = pairs / 4;
    if (want < 2) return 1;
    const uint32_t pairs_per = (uint32_t)((pairs + want - 1) / want);
    *ksplit = pairs_per * pair_elems;
    return (g.K + *ksplit - 1) / *ksplit;
}

// Bytes of fp32 partials a split K range of this product needs ([split][batch][M][N]), 0 when the
// tile kernel would not split it or the skinny kernel takes it with 16-byte aligned operands.  (A
// skinny-shaped product with misaligned operands goes to the tile kernel, and runs unsplit when
// the workspace sized here is 0.)
template <int DT>
size_t split_bytes(const GemmArgs& g) {
    using S = typename MmaTraits<DT>::S;
    alignas(16) static const char aligned[16] = {};
    if (skinny_ok<DT>(g, aligned, aligned)) return 0;
    if (skinny_nn_ok<DT>(g, aligned, aligned)) {
        const uint64_t per = (uint64_t)g.batches * g.M * g.N;
        const uint32_t nsplit = skinny_nn_splits<DT>(g);
        return nsplit > 1 && per < 0xffffffffull ? (size_t)nsplit * per * sizeof(float) : 0;
    }
    const tile::TileShape ts = tile_for<DT>(g);
    uint32_t ksplit = 0;
    const uint32_t nsplit = choose_split(ts, g, tile::ROWB / sizeof(S), &ksplit);
    const uint64_t per = (uint64_t)g.batches * g.M * g.N;
    return nsplit > 1 && per < 0xffffffffull ? (size_t)nsplit * per * sizeof(float) : 0;
}

// ws / ws_bytes: the caller's workspace for split-K partials.  A product whose split needs more
// than ws_bytes (none given: 0) runs unsplit; nothing here allocates.
template <int DT>
int launch_mfma(GemmArgs& g, void* C, const void* A, const void* Bt, void* ws, size_t ws_bytes, hipStream_t st,
                const Epi* epi = nullptr) {
    using S = typename MmaTraits<DT>::S;
    constexpr int CE = 16 / sizeof(S);
    if (skinny_ok<DT>(g, A, Bt)) {
        const int rc = launch_skinny<DT>(g, C, A, Bt, st);
        return rc || !epi ? rc : launch_bias_act<DT>(g, C, *epi, st);
    }
    if (skinny_nn_ok<DT>(g, A, Bt)) {
        using P = SkinnyNN<DT>;
        const uint64_t per = (uint64_t)g.batches * g.M * g.N;
        uint32_t nsplit = skinny_nn_splits<DT>(g);
        if (nsplit > 1 && (ws == nullptr || (uintptr_t)ws % 16 || per >= 0xffffffffull ||
                           (size_t)nsplit * per * sizeof(float) > ws_bytes))
            nsplit = 1;
        uint32_t kw = (uint32_t)((g.K + (uint64_t)nsplit * P::W - 1) / ((uint64_t)nsplit * P::W));
        kw = (kw + P::KS - 1) / P::KS * P::KS;
        const uint32_t ncg = (g.N + P::NC - 1) / P::NC;
        if ((uint64_t)ncg * nsplit > 0x7fffffffull) return fail(MX_ERR_INVALID_ARG, "mx_launch_batched_matmul: grid too large");
        const dim3 grid(ncg * nsplit, g.batches), block(64 * P::W);
        if (nsplit == 1) {
            hipLaunchKernelGGL((gemm_skinny_nn_kernel<DT, false>), grid, block, 0, st, C, (const S*)A, (const S*)Bt, g,
                               ncg, kw);
            MX_HIP(hipGetLastError());
            return epi ? launch_bias_act<DT>(g, C, *epi, st) : MX_OK;
        }
        hipLaunchKernelGGL((gemm_skinny_nn_kernel<DT, true>), grid, block, 0, st, ws, (const S*)A, (const S*)Bt, g, ncg,
                           kw);
        MX_HIP(hipGetLastError());
        const dim3 sgrid((uint32_t)((per + 255) / 256));
        if (epi)
            hipLaunchKernelGGL((splitk_sum_kernel<DT, true>), sgrid, dim3(256), 0, st, (S*)C, (const float*)ws, nsplit,
                               g, FastDiv(g.N), FastDiv(g.M), *epi);
        else
            hipLaunchKernelGGL((splitk_sum_kernel<DT, false>), sgrid, dim3(256), 0, st, (S*)C, (const float*)ws, nsplit,
                               g, FastDiv(g.N), FastDiv(g.M), Epi{});
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    const tile::TileShape ts = tile_for<DT>(g);
    uint32_t ksplit = 0;
    uint32_t nsplit = choose_split(ts, g, tile::ROWB / sizeof(S), &ksplit);
    const uint64_t per = (uint64_t)g.batches * g.M * g.N;
    if (nsplit > 1 && (ws == nullptr || (size_t)nsplit * per * sizeof(float) > ws_bytes)) nsplit = 1;
    // the DMA path addresses a tile's rows with 32-bit byte offsets
    const bool vec = g.ka == 1 && g.kb == 1 && g.lda % CE == 0 && g.ldb % CE == 0 &&
                     (uint64_t)ts.bm * g.lda * sizeof(S) < (1ull << 32) &&
                     (uint64_t)ts.bn * g.ldb * sizeof(S) < (1ull << 32) &&
                     (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 && [&] {
                         for (int d = 0; d < g.bd.n; d++)
                             if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
                         return true;
                     }();
    // B given N-major (Bt's K stride is B's row stride, its N stride 1): the tile kernel's N-major
    // B slot (fp32: 16-byte rows of 4 columns; 16-bit: transposing LDS reads), so dot() needs no
    // transposed copy of B
    const bool nn = !vec && g.ka == 1 && g.ldb == 1 && g.kb % CE == 0 && g.N % CE == 0 && g.lda % CE == 0 &&
                    (uint64_t)ts.bm * g.lda * sizeof(S) < (1ull << 32) && 64ull * g.kb * sizeof(S) < (1ull << 32) &&
                    (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 && [&] {
                        for (int d = 0; d < g.bd.n; d++)
                            if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
                        return true;
                    }();
    // A given M-major (A's K stride is its row pitch, its M stride 1: the vjp's g^T): the A slot
    // takes B's N-major layout (16-bit: transposing reads; fp32: Frags32T), so dot() needs no copy
    // of g^T.  B either K-major (the DMA path's Bt) or N-major.
    const bool bk = g.kb == 1 && g.ldb % CE == 0 && (uint64_t)ts.bn * g.ldb * sizeof(S) < (1ull << 32);
    const bool bn = g.ldb == 1 && g.kb % CE == 0 && g.N % CE == 0 && 64ull * g.kb * sizeof(S) < (1ull << 32);
    const bool amn = g.lda == 1 && g.ka % CE == 0 && g.M % CE == 0 &&
                     64ull * g.ka * sizeof(S) < (1ull << 32) && (bk || bn) && (uintptr_t)A % 16 == 0 &&
                     (uintptr_t)Bt % 16 == 0 && [&] {
                         for (int d = 0; d < g.bd.n; d++)
                             if (g.bd.sA[d] % CE || g.bd.sB[d] % CE) return false;
                         return true;
                     }();
    const tile::MatrixSrc::Geom geo{};
    const char* who = "mx_launch_batched_matmul";
    // the tile kernel for this layout: (K-major | M-major A) x (K-major | N-major B), or strided
    auto tile_launch = [&](auto split, GemmArgs& ga, void* out, uint32_t ns) -> int {
        constexpr bool SP = decltype(split)::value;
        if (amn && bn) return tile::launch_tile_kernel<DT, true, SP, tile::MatrixSrc, true, true>(ts, ga, geo, out, A, Bt, st, who, ns);
        if (amn) return tile::launch_tile_kernel<DT, true, SP, tile::MatrixSrc, false, true>(ts, ga, geo, out, A, Bt, st, who, ns);
        if (nn) return tile::launch_tile_kernel<DT, true, SP, tile::MatrixSrc, true>(ts, ga, geo, out, A, Bt, st, who, ns);
        return vec ? tile::launch_tile_kernel<DT, true, SP, tile::MatrixSrc>(ts, ga, geo, out, A, Bt, st, who, ns)
                   : tile::launch_tile_kernel<DT, false, SP, tile::MatrixSrc>(ts, ga, geo, out, A, Bt, st, who, ns);
    };
    if (nsplit > 1 && per < 0xffffffffull) {
        // fp32 partials [split][batch][M][N] in the caller's workspace, then an ordered sum
        void* P = ws;
        int rc = MX_OK;
        GemmArgs gp = g;
        gp.ksplit = ksplit;
        gp.ldc = g.N;
        gp.cn = 1;
        rc = tile_launch(std::true_type{}, gp, P, nsplit);
        if (rc) return rc;
        const dim3 grid((uint32_t)((per + 255) / 256));
        if (epi)
            hipLaunchKernelGGL((splitk_sum_kernel<DT, true>), grid, dim3(256), 0, st, (S*)C, (const float*)P, nsplit, g,
                               FastDiv(g.N), FastDiv(g.M), *epi);
        else
            hipLaunchKernelGGL((splitk_sum_kernel<DT, false>), grid, dim3(256), 0, st, (S*)C, (const float*)P, nsplit, g,
                               FastDiv(g.N), FastDiv(g.M), Epi{});
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    const int rc = tile_launch(std::false_type{}, g, C, 1);
    return rc || !epi ? rc : launch_bias_act<DT>(g, C, *epi, st);
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

namespace {

// Fills g from the collapsed descriptor (mx_launch_batched_matmul's arguments).  Returns MX_OK,
// a failure status, or -1 when there is nothing to compute.
int matmul_args(const char* who, int cdims, const uint32_t* shapeC, const uint32_t* sA, const uint32_t* sBt,
                const uint32_t* sC, uint32_t K, void* C, const void* A, const void* Bt, GemmArgs& g) {
    if (cdims < 2 || cdims > MX_MAX_DIMS)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": cdims " + std::to_string(cdims) + " outside [2, 8]");
    if (!shapeC || !sA || !sBt || !sC) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null descriptor");
    g = GemmArgs{};
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
    if (batches == 0 || g.M == 0 || g.N == 0) return -1;
    if (batches * g.M > 0xffffffffull || batches * g.N > 0xffffffffull)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": extent above 2^32-1 (size_m indexing)");
    if (!C || ((!A || !Bt) && K > 0)) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null buffer");
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
    return MX_OK;
}

}  // namespace

namespace {

int launch_any(int dtype, GemmArgs& g, void* C, const void* A, const void* Bt, void* ws, size_t ws_bytes,
               hipStream_t st) {
    switch (dtype) {
    case MX_FLOAT32: return launch_mfma<MX_FLOAT32>(g, C, A, Bt, ws, ws_bytes, st);
    case MX_FLOAT16: return launch_mfma<MX_FLOAT16>(g, C, A, Bt, ws, ws_bytes, st);
    case MX_BFLOAT16: return launch_mfma<MX_BFLOAT16>(g, C, A, Bt, ws, ws_bytes, st);
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

}  // namespace

extern "C" int mx_matmul_workspace_bytes(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                                         const uint32_t* sBt, const uint32_t* sC, uint32_t K, size_t* bytes) {
    if (!bytes) return fail(MX_ERR_INVALID_ARG, "mx_matmul_workspace_bytes: null out pointer");
    *bytes = 0;
    GemmArgs g;
    // buffers are not needed to size the workspace: pass a placeholder so the null check passes
    static const char dummy[16] = {};
    const int ar = matmul_args("mx_matmul_workspace_bytes", cdims, shapeC, sA, sBt, sC, K, (void*)dummy, dummy,
                               dummy, g);
    if (ar) return ar < 0 ? MX_OK : ar;
    switch (dtype) {
    case MX_FLOAT32: *bytes = split_bytes<MX_FLOAT32>(g); return MX_OK;
    case MX_FLOAT16: *bytes = split_bytes<MX_FLOAT16>(g); return MX_OK;
    case MX_BFLOAT16: *bytes = split_bytes<MX_BFLOAT16>(g); return MX_OK;
    case MX_INT32: case MX_INT16: case MX_INT8: case MX_INT64: case MX_UINT8: case MX_UINT16: case MX_UINT32:
    case MX_UINT64: case MX_BOOL: return MX_OK;
    default:
        return fail(MX_ERR_UNSUPPORTED, "mx_matmul_workspace_bytes: no kernel for dtype " + std::to_string(dtype));
    }
}

extern "C" int mx_launch_batched_matmul_ws(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                                           const uint32_t* sBt, const uint32_t* sC, uint32_t K, void* C,
                                           const void* A, const void* Bt, void* workspace, size_t workspace_bytes,
                                           void* stream) {
    GemmArgs g;
    const int ar = matmul_args("mx_launch_batched_matmul", cdims, shapeC, sA, sBt, sC, K, C, A, Bt, g);
    if (ar) return ar < 0 ? MX_OK : ar;
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    return launch_any(dtype, g, C, A, Bt, workspace, workspace ? workspace_bytes : 0, st);
}

extern "C" int mx_launch_batched_matmul(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                                        const uint32_t* sBt, const uint32_t* sC, uint32_t K, void* C,
                                        const void* A, const void* Bt, void* stream) {
    return mx_launch_batched_matmul_ws(dtype, cdims, shapeC, sA, sBt, sC, K, C, A, Bt, nullptr, 0, stream);
}

extern "C" int mx_launch_batched_matmul_bias_act(int dtype, int cdims, const uint32_t* shapeC, const uint32_t* sA,
                                                 const uint32_t* sBt, const uint32_t* sC, uint32_t K, void* C,
                                                 const void* A, const void* Bt, const void* bias, void* Z,
                                                 int act_op, const void* act_scalar, void* H, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
    const char* who = "mx_launch_batched_matmul_bias_act";
    if (dtype != MX_FLOAT32 && dtype != MX_FLOAT16 && dtype != MX_BFLOAT16)
        return fail(MX_ERR_UNSUPPORTED, std::string(who) + ": float32 / float16 / bfloat16 only, dtype " +
                                            std::to_string(dtype));
    if (act_op != MX_OP_MAX && act_op != MX_OP_MIN)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": act_op must be MX_OP_MAX or MX_OP_MIN");
    GemmArgs g;
    const int ar = matmul_args(who, cdims, shapeC, sA, sBt, sC, K, C, A, Bt, g);
    if (ar) return ar < 0 ? MX_OK : ar;
    // C (and so Z and H) contiguous: the epilogue walks them linearly
    uint64_t want = 1;
    for (int d = cdims - 1; d >= 0; --d) {
        if (shapeC[d] != 1 && sC[d] != want)
            return fail(MX_ERR_INVALID_ARG, std::string(who) + ": C must be contiguous");
        want *= shapeC[d];
    }
    if (want > 0xffffffffull) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": more than 2^32-1 outputs");
    if (!bias || !Z || !act_scalar || !H) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    const Epi e{Z, H, bias, act_scalar, act_op};
    const size_t wsb = workspace ? workspace_bytes : 0;
    switch (dtype) {
    case MX_FLOAT32: return launch_mfma<MX_FLOAT32>(g, C, A, Bt, workspace, wsb, st, &e);
    case MX_FLOAT16: return launch_mfma<MX_FLOAT16>(g, C, A, Bt, workspace, wsb, st, &e);
    default: return launch_mfma<MX_BFLOAT16>(g, C, A, Bt, workspace, wsb, st, &e);
    }
}
