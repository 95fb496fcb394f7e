// mfma_tile.hpp -- the CDNA4 matrix-core tile kernel shared by batched MatMul (gemm.hip) and
// ConvolutionND as an implicit GEMM (conv.hip).
//
// C[b, m, n] = sum_k A[b, m, k] * Bt[b, n, k], both operands K-major (the layout the reference
// hands its backends: dot() packs B^T, Matrix.mm:7074-7089; the conv kernel is OHWI,
// Matrix.mm:12274-12277).  float16 / bfloat16: v_mfma_f32_32x32x16_{f16,bf16}, fp32
// accumulation, one rounding on store.  float32: v_mfma_f32_32x32x2_f32.
//
// Tiling: a block computes a BM x BN tile of C (each 256 or 128) as 2 x WN waves of BM/2 x BN/WN
// (BM/64 x BN/(32 WN) MFMA tiles of 32 x 32 per wave, fp32 accumulators): WN = 2 (256 threads),
// or WN = 4 (512 threads) for 16-bit 256 x 256 and 128 x 128 tiles and fp32 ones with A K-major.
// A K step
// covers 64 bytes of each row (32 elements of 16-bit data, 16 of fp32); LDS holds two slots of a
// K pair -- 128 bytes of every row of A and of Bt -- so every fetch is a whole 128-byte line
// (half-line fetches doubled the L2 -> LDS traffic).  Direct global -> LDS loads (gfx950
// buffer_load_dwordx4 ... lds) fill the slot of pair p + 2 while pair p + 1 is consumed; fragments
// are double-buffered in registers, and the workgroup meets one barrier per pair.  Each slot is
// its own __shared__ array, so the compiler can tell the DMA into one slot from the reads of the
// other and adds no waits of its own.  LDS rows are 8 chunks of 16 bytes, swizzled so that one
// MFMA operand read is bank-conflict free.  Block ids are remapped so that the tiles one XCD
// (one L2) runs are consecutive M panels with all their N tiles.
//
// Where the A rows come from is a policy (Src): a strided matrix (GEMM) or an on-the-fly
// im2col gather from a channels-last image (implicit-GEMM convolution), whose out-of-image
// taps read zeros.  The same policy maps a C row to its output offset.
#pragma once
#include "common.hpp"

namespace mx {
namespace tile {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef __bf16 b8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
// fp32 fragments are native 4-wide vectors: loaded through HIP's float4 struct, the LDS reads lost
// the alias scopes that tell them apart from the DMA into the other slot, and the compiler then
// made them wait for that DMA.
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int STEPB = 64;                 // bytes of K per row in one K step (one MFMA round)
constexpr int ROWB = 2 * STEPB;           // bytes of one LDS row: a K pair, one 128-byte line
constexpr int CPR = ROWB / 16;            // 16-byte chunks per LDS row
constexpr int STEP_CHUNKS = STEPB / 16;
constexpr int NTHREADS = 256;
constexpr int NUM_XCD = 8;
template <int ROWS, int NW = 4> constexpr int kDma = ROWS * ROWB / 1024 / NW;   // 1 KB DMAs per wave per slot

template <int DT> struct MmaTraits;
template <> struct MmaTraits<MX_FLOAT16> { using S = uint16_t; };
template <> struct MmaTraits<MX_BFLOAT16> { using S = uint16_t; };
template <> struct MmaTraits<MX_FLOAT32> { using S = float; };

struct BatchDesc {                // batch axes (all but the last two of a collapsed descriptor)
    int n;
    FastDiv shape[MX_MAX_DIMS];
    uint32_t sA[MX_MAX_DIMS], sB[MX_MAX_DIMS], sC[MX_MAX_DIMS];
};

struct GemmArgs {
    uint32_t M, N, K;
    uint32_t lda, ldb;            // row strides (elements) of A [M, K] and Bt [N, K]
    uint32_t ka, kb;              // K strides of A and Bt (1 on the DMA path)
    uint32_t ldc, cn;             // C strides: row (M) and column (N)
    uint32_t tiles_m, tiles_n, batches;
    uint32_t ksplit;              // split-K: K elements per split (the split kernels only)
    BatchDesc bd;
};

// LDS swizzle: logical chunk c of row r is stored at c ^ ((r >> 1) & 7).  The LDS serves a
// 128-bit read 16 lanes (256 bytes, 64 banks) at a time; one MFMA operand read has 16 lanes on
// 16 consecutive rows with the same logical chunk, whose 16-byte bank groups
// 8 (r % 2) + stored chunk are then all distinct.
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Block id -> (batch, tile_m, tile_n).  Hardware dispatch hands block i to XCD i % 8; the
// remap gives each XCD a contiguous run of logical tiles, ordered M panel by M panel.
__device__ __forceinline__ void tile_of(uint32_t id, uint32_t nblocks, uint32_t tiles_m, uint32_t tiles_n,
                                        uint32_t& b, uint32_t& tm, uint32_t& tn) {
    const uint32_t per = nblocks / NUM_XCD, rem = nblocks % NUM_XCD;
    const uint32_t x = id % NUM_XCD, j = id / NUM_XCD;
    const uint32_t logical = (x < rem) ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
    const uint32_t tiles = tiles_m * tiles_n;
    b = logical / tiles;
    const uint32_t t = logical - b * tiles;
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
}

// K tail or strided operands: one K step (the first half of an LDS row) of a ROWS-row tile
// through registers, element loads, zero past K (zeros keep the tail exact).  This thread's
// chunk q = tid + 256 i is row q / 4, logical chunk q % 4.  Rows past the operand's end re-read
// its last row (their products land only in C rows / columns that are never stored).
template <int ROWS, int NT = NTHREADS> constexpr int kTailChunks = ROWS * STEP_CHUNKS / NT;

template <typename S, int ROWS, int NT = NTHREADS>
__device__ __forceinline__ void load_tile_guarded(uint4 (&r)[(kTailChunks<ROWS, NT>)], const S* __restrict__ base,
                                                  uint32_t rows_valid, uint32_t ld, uint32_t kstride, uint32_t k0,
                                                  uint32_t K) {
    constexpr int CE = 16 / sizeof(S);
#pragma unroll
    for (int i = 0; i < kTailChunks<ROWS, NT>; i++) {
        const int q = threadIdx.x + NT * i;
        const uint32_t row = min((uint32_t)(q / STEP_CHUNKS), rows_valid - 1);
        const uint32_t k = k0 + (q % STEP_CHUNKS) * CE;
        S tmp[CE];
#pragma unroll
        for (int e = 0; e < CE; e++)
            tmp[e] = (k + e < K) ? base[(uint64_t)row * ld + (uint64_t)(k + e) * kstride] : S(0);
        __builtin_memcpy(&r[i], tmp, 16);
    }
}

template <int ROWS, int NT = NTHREADS>
__device__ __forceinline__ void store_tile(char* lds, const uint4 (&r)[(kTailChunks<ROWS, NT>)]) {
#pragma unroll
    for (int i = 0; i < kTailChunks<ROWS, NT>; i++) {
        const int q = threadIdx.x + NT * i;
        const int row = q / STEP_CHUNKS, c = q % STEP_CHUNKS;
        *reinterpret_cast<uint4*>(lds + row * ROWB + swz(row, c) * 16) = r[i];
    }
}

// One K step's operand fragments for one wave (TM A tiles, WNT Bt tiles of 32 rows).  The step
// is half HALF of the LDS rows (logical chunks 4 HALF .. 4 HALF + 3).  16-bit types: a K block
// is 16 elements = 2 chunks; lane half h holds chunk 2 kb + h of the step.  fp32: the step is
// one K block of 16 elements = 4 chunks; lane half h holds chunks 2h, 2h + 1 (K offsets
// 8h .. 8h + 7); MFMA substep s consumes element s, so the two lane halves supply k = s and
// k = 8 + s.
template <int DT, int TM, int WNT> struct Frags;
template <int TM, int WNT> struct Frags<MX_FLOAT16, TM, WNT> { static constexpr int KB = 2; h8v a[KB][TM], b[KB][WNT]; };
template <int TM, int WNT> struct Frags<MX_BFLOAT16, TM, WNT> { static constexpr int KB = 2; b8v a[KB][TM], b[KB][WNT]; };
template <int TM, int WNT> struct Frags<MX_FLOAT32, TM, WNT> {
    static constexpr int KB = 1;
    f4v a[KB][TM][2], b[KB][WNT][2];
};

template <int DT, int TM, int WNT, int HALF>
__device__ __forceinline__ void read_frags(Frags<DT, TM, WNT>& f, const char* la, const char* lb, int wm, int wn,
                                           int lane) {
    const int r32 = lane & 31, h = lane >> 5;
    constexpr int C0 = HALF * STEP_CHUNKS;
#pragma unroll
    for (int kb = 0; kb < Frags<DT, TM, WNT>::KB; kb++) {
#pragma unroll
        for (int t = 0; t < TM; t++) {
            const int ra = wm * (TM * 32) + t * 32 + r32;
            if constexpr (DT == MX_FLOAT32) {
#pragma unroll
                for (int u = 0; u < 2; u++)
                    f.a[kb][t][u] = *reinterpret_cast<const f4v*>(la + ra * ROWB + swz(ra, C0 + 2 * h + u) * 16);
            } else {
                using V = std::remove_reference_t<decltype(f.a[0][0])>;
                f.a[kb][t] = *reinterpret_cast<const V*>(la + ra * ROWB + swz(ra, C0 + 2 * kb + h) * 16);
            }
        }
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int rb = wn * (WNT * 32) + t * 32 + r32;
            if constexpr (DT == MX_FLOAT32) {
#pragma unroll
                for (int u = 0; u < 2; u++)
                    f.b[kb][t][u] = *reinterpret_cast<const f4v*>(lb + rb * ROWB + swz(rb, C0 + 2 * h + u) * 16);
            } else {
                using V = std::remove_reference_t<decltype(f.b[0][0])>;
                f.b[kb][t] = *reinterpret_cast<const V*>(lb + rb * ROWB + swz(rb, C0 + 2 * kb + h) * 16);
            }
        }
    }
}

__device__ __forceinline__ float f4_at(const f4v (&v)[2], int s) { return v[s >> 2][s & 3]; }

// MFMAs of the step for A tile rows I0 .. I1 - 1 of the wave's TM x WNT grid.  The Bt fragment
// goes in the MFMA's first operand slot and the A fragment in the second, so the 32 x 32 result
// is the C^T tile: lane l holds C row (l % 32) and, in acc[4 q .. 4 q + 3], the 4 consecutive C
// columns 8 q + 4 (l / 32) .. + 3 -- one vector store per (q) in the epilogue.
template <int DT, int TM, int WNT, int I0, int I1>
__device__ __forceinline__ void mma_step(f16v (&acc)[TM][WNT], const Frags<DT, TM, WNT>& f) {
#pragma unroll
    for (int kb = 0; kb < Frags<DT, TM, WNT>::KB; kb++) {
        if constexpr (DT == MX_FLOAT32) {
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int i = I0; i < I1; i++)
#pragma unroll
                    for (int j = 0; j < WNT; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f4_at(f.b[kb][j], s), f4_at(f.a[kb][i], s),
                                                                        acc[i][j], 0, 0, 0);
        } else {
#pragma unroll
            for (int i = I0; i < I1; i++)
#pragma unroll
                for (int j = 0; j < WNT; j++) {
                    if constexpr (DT == MX_FLOAT16)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.b[kb][j], f.a[kb][i], acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[kb][j], f.a[kb][i], acc[i][j], 0, 0, 0);
                }
        }
    }
}

// fp32 with Bt N-major (B given as [K, N], N contiguous -- dot()'s B without its transposed copy).
// The B slot holds the pair's 32 K rows of BN floats.  The wave's WNT x 32 columns are read as 32
// groups of WNT consecutive columns: lane (i = l % 32, h = l / 32) loads, for substep s, row 8 h + s
// (the K offset the A fragment of lane half h holds, see Frags) and columns WNT i .. WNT i + WNT - 1,
// and MFMA q of the substep takes element q as its row operand.  MFMA q thus covers the columns
// n = WNT i + q: C^T row i of accumulator q is column WNT i + q, so a lane's WNT accumulators hold
// WNT consecutive columns (one vector store in the epilogue).
template <int TM, int WNT> struct FragsNN {
    static constexpr int KB = 1;
    typedef float bvec __attribute__((ext_vector_type(WNT)));
    f4v a[1][TM][2];
    bvec b[8];
};

template <int TM, int WNT, int BN, int HALF>
__device__ __forceinline__ void read_frags_nn(FragsNN<TM, WNT>& f, const char* la, const char* lb, int wm, int wn,
                                              int lane) {
    using BV = typename FragsNN<TM, WNT>::bvec;
    const int r32 = lane & 31, h = lane >> 5;
    constexpr int C0 = HALF * STEP_CHUNKS;
#pragma unroll
    for (int t = 0; t < TM; t++) {
        const int ra = wm * (TM * 32) + t * 32 + r32;
#pragma unroll
        for (int u = 0; u < 2; u++)
            f.a[0][t][u] = *reinterpret_cast<const f4v*>(la + ra * ROWB + swz(ra, C0 + 2 * h + u) * 16);
    }
    const int col = wn * (WNT * 32) + WNT * r32;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int row = HALF * 16 + 8 * h + s;
        f.b[s] = *reinterpret_cast<const BV*>(lb + row * (BN * 4) + col * 4);
    }
}

template <int TM, int WNT, int I0, int I1>
__device__ __forceinline__ void mma_step_nn(f16v (&acc)[TM][WNT], const FragsNN<TM, WNT>& f) {
#pragma unroll
    for (int s = 0; s < 8; s++)
#pragma unroll
        for (int i = I0; i < I1; i++)
#pragma unroll
            for (int q = 0; q < WNT; q++)
                acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.b[s][q], f4_at(f.a[0][i], s), acc[i][q], 0, 0, 0);
}

// fp32 with A M-major (A as [K, M], M contiguous: the vjp's g^T), and B K- or N-major.  The A slot
// holds the pair's 32 K rows of BM floats, read like the N-major B slot: lane (i = l % 32, h)
// loads, for substep s, row 8 h + s and rows TM i .. TM i + TM - 1 of the wave's A range, and the
// MFMA of A tile t takes element t -- so accumulator t holds C row TM (l % 32) + t of the wave's
// range (the epilogue maps rows accordingly) instead of 32 t + l % 32.
template <int TM, int WNT, bool BT> struct Frags32T {
    static constexpr int KB = 1;
    typedef float avec __attribute__((ext_vector_type(TM)));
    typedef float bvec __attribute__((ext_vector_type(WNT)));
    avec a[8];
    f4v bk[1][WNT][2];                     // B K-major (BT false)
    bvec bn[8];                            // B N-major (BT true)
};

template <int TM, int WNT, int BM, int BN, int HALF, bool BT>
__device__ __forceinline__ void read_frags_32t(Frags32T<TM, WNT, BT>& f, const char* la, const char* lb, int wm, int wn,
                                               int lane) {
    using AV = typename Frags32T<TM, WNT, BT>::avec;
    using BV = typename Frags32T<TM, WNT, BT>::bvec;
    const int r32 = lane & 31, h = lane >> 5;
    const int acol = wm * (TM * 32) + TM * r32;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int row = HALF * 16 + 8 * h + s;
        f.a[s] = *reinterpret_cast<const AV*>(la + row * (BM * 4) + acol * 4);
    }
    if constexpr (BT) {
        const int col = wn * (WNT * 32) + WNT * r32;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int row = HALF * 16 + 8 * h + s;
            f.bn[s] = *reinterpret_cast<const BV*>(lb + row * (BN * 4) + col * 4);
        }
    } else {
        constexpr int C0 = HALF * STEP_CHUNKS;
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int rb = wn * (WNT * 32) + t * 32 + r32;
#pragma unroll
            for (int u = 0; u < 2; u++)
                f.bk[0][t][u] = *reinterpret_cast<const f4v*>(lb + rb * ROWB + swz(rb, C0 + 2 * h + u) * 16);
        }
    }
}

template <int TM, int WNT, int I0, int I1, bool BT>
__device__ __forceinline__ void mma_step_32t(f16v (&acc)[TM][WNT], const Frags32T<TM, WNT, BT>& f) {
#pragma unroll
    for (int s = 0; s < 8; s++)
#pragma unroll
        for (int i = I0; i < I1; i++)
#pragma unroll
            for (int q = 0; q < WNT; q++) {
                if constexpr (BT)
                    acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.bn[s][q], f.a[s][i], acc[i][q], 0, 0, 0);
                else
                    acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x2f32(f4_at(f.bk[0][q], s), f.a[s][i], acc[i][q], 0, 0, 0);
            }
}

// Direct global -> LDS copy of one operand's K pair (two steps, 128 bytes of each row -- whole
// L2 lines).  Each of a wave's DMA instructions fills 1 KB = 8 LDS rows; lane L lands at row
// r = 8 p + L / 8, stored chunk L % 8, so it fetches the logical chunk that swz() stores there
// (swz is its own inverse).  For a strided matrix the lane's byte offsets from the tile's first
// row are fixed for the whole K loop; each pair adds its K offset to the wave-uniform base.
// The offsets are 32-bit: the launcher keeps the tile's rows below 4 GiB.
template <int N> struct DmaOffsets { uint32_t v[N]; };

__device__ __forceinline__ int dma_row(int wave, int i, int per_wave, int lane) {
    return (wave * per_wave + i) * 8 + lane / CPR;
}
__device__ __forceinline__ int dma_chunk(int row, int lane) { return swz(row, lane % CPR); }

template <typename S, int N>
__device__ __forceinline__ DmaOffsets<N> dma_offsets(uint32_t rows_valid, uint32_t ld, int wave, int lane) {
    constexpr int CE = 16 / sizeof(S);
    DmaOffsets<N> o;
#pragma unroll
    for (int i = 0; i < N; i++) {
        const int r = dma_row(wave, i, N, lane);
        const uint32_t row = min((uint32_t)r, rows_valid - 1);
        o.v[i] = (row * ld + dma_chunk(r, lane) * CE) * (uint32_t)sizeof(S);
    }
    return o;
}

__device__ __forceinline__ void dma16(const void* src, char* lds_chunk_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_chunk_base, 16, 0, 0);
}

// A matrix operand's rows go through the buffer form of the LDS DMA (buffer_load_dwordx4 ... lds,
// a raw resource at the wave-uniform base, no range limit, the lane offset in a VGPR).  The
// compiler counts that form in vmcnt only, so the fragment reads after a DMA wait for just the
// reads they need; with the global form (a FLAT instruction that may also count in lgkmcnt) it
// waits for every outstanding LDS read first (lgkmcnt(0)).  f16 main GEMM +1-3%, f16 3x3
// convolution 26.9 -> 26.2 us.
template <typename S, int N>
__device__ __forceinline__ void dma_rows(char* lds, const S* __restrict__ base, const DmaOffsets<N>& o, uint32_t k0,
                                         int wave) {
#if __HIP_DEVICE_COMPILE__                               // (the buffer resource type is device-only)
    const char* kbase = reinterpret_cast<const char*>(base + k0);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kbase), 0, -1, 0x00020000);
#pragma unroll
    for (int i = 0; i < N; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds + (wave * N + i) * 1024),
                                                 16, o.v[i], 0, 0, 0);
#endif
}

// B slot of the N-major layout: one DMA instruction fills 1 KB = 1024 / (4 BN) K rows; wave w's
// instruction i fills rows RPI (DMA_B w + i) ..  Columns past N load the last whole vector of the
// row (their products land only in C columns that are never stored); N is a multiple of 4 here.
template <int BN, int N>
__device__ __forceinline__ DmaOffsets<N> dma_offsets_nn(uint32_t cols_valid, uint32_t ldk, int wave, int lane) {
    constexpr int RPI = 1024 / (BN * 4);                 // rows per DMA instruction
    constexpr int LPR = 64 / RPI;                        // lanes per row
    DmaOffsets<N> o;
#pragma unroll
    for (int i = 0; i < N; i++) {
        const uint32_t row = (uint32_t)((wave * N + i) * RPI + lane / LPR);
        const uint32_t col = min((uint32_t)(lane % LPR) * 4, cols_valid - 4);
        o.v[i] = (row * ldk + col) * 4u;
    }
    return o;
}

// One K step (16 rows) of the N-major B tile through registers, element loads, zero past K; rows
// 0 .. 15 of the slot.  Thread chunk q = tid + 256 j is row q / (BN / 4), columns 4 (q % (BN / 4)).
template <int BN, int NT = NTHREADS> constexpr int kTailChunksNN = 16 * BN / 4 / NT;

template <int BN, int NT = NTHREADS>
__device__ __forceinline__ void load_tile_guarded_nn(f4v (&r)[(kTailChunksNN<BN, NT>)], const float* __restrict__ base,
                                                     uint32_t cols_valid, uint32_t ldk, uint32_t k0, uint32_t K) {
#pragma unroll
    for (int j = 0; j < kTailChunksNN<BN, NT>; j++) {
        const int q = threadIdx.x + NT * j;
        const uint32_t k = k0 + (uint32_t)(q / (BN / 4));
        const uint32_t c = (uint32_t)(q % (BN / 4)) * 4;
#pragma unroll
        for (int e = 0; e < 4; e++)
            r[j][e] = (k < K && c + e < cols_valid) ? base[(uint64_t)k * ldk + c + e] : 0.0f;
    }
}

template <int BN, int NT = NTHREADS>
__device__ __forceinline__ void store_tile_nn(char* lds, const f4v (&r)[(kTailChunksNN<BN, NT>)]) {
#pragma unroll
    for (int j = 0; j < kTailChunksNN<BN, NT>; j++) {
        const int q = threadIdx.x + NT * j;
        *reinterpret_cast<f4v*>(lds + (q / (BN / 4)) * (BN * 4) + (q % (BN / 4)) * 16) = r[j];
    }
}

// ------------------------------------------------------------------ 16-bit B given N-major
// B as [K, N] with N contiguous (dot()'s B without its transposed copy).  The B slot holds the
// pair's 64 K rows of BN elements (BN * 2 bytes each); 16-byte chunk c of K row k is stored at
// c ^ (4 (k & 3)).  A fragment (8 consecutive K of one column, as the K-major slot gives it) comes
// from two transposing LDS reads (ds_read_b64_tr_b16).  Within each group of 16 lanes, that read
// takes a 4 x 16 block of 16-bit elements whose row e is the four 8-byte pieces addressed by lanes
// 4e .. 4e + 3 (lane 4e + q: columns 4q .. 4q + 3), and returns column i of the block to lane i: so
// lane 4e + q addresses K row kb + e, columns nb + 4q .. + 3, and lane i receives rows kb .. kb + 3
// of column nb + i.  The swizzle puts the eight 32-byte row segments two lane groups read at once
// (K rows kb .. kb + 3, columns nb and nb + 16) in eight distinct groups of LDS banks.
__device__ __forceinline__ int swz_nn16(int krow, int chunk) { return chunk ^ (4 * (krow & 3)); }

typedef short s4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ s4v ds_read_tr16(const char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4v*)((__attribute__((address_space(3))) char*)p));
}

// The Bt fragment of lane l for MFMA column tile t, K block kb of step HALF: lane l holds column
// n = wn * 32 WNT + 32 t + l % 32 and K offsets 16 kb + 8 (l / 32) .. + 7 of the step, as
// read_frags gives it from a K-major slot.
template <int BN, int HALF, typename V>
__device__ __forceinline__ V read_b_nn16(const char* lb, int col0, int kb, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const int krow = HALF * 32 + 16 * kb + 8 * (g >> 1) + (j >> 2);
    const int col = col0 + 16 * (g & 1) + 4 * (j & 3);
    const int c = col >> 3, half8 = (col & 7) * 2;          // 16-byte chunk, byte offset in it
    const s4v lo = ds_read_tr16(lb + krow * (BN * 2) + swz_nn16(krow, c) * 16 + half8);
    const s4v hi = ds_read_tr16(lb + (krow + 4) * (BN * 2) + swz_nn16(krow + 4, c) * 16 + half8);
    const auto v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    V out;
    __builtin_memcpy(&out, &v, 16);
    return out;
}

template <int DT, int TM, int WNT, int BN, int HALF>
__device__ __forceinline__ void read_frags_nn16(Frags<DT, TM, WNT>& f, const char* la, const char* lb, int wm, int wn,
                                                int lane) {
    using V = std::remove_reference_t<decltype(f.b[0][0])>;
    const int r32 = lane & 31, h = lane >> 5;
    constexpr int C0 = HALF * STEP_CHUNKS;
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
#pragma unroll
        for (int t = 0; t < TM; t++) {
            const int ra = wm * (TM * 32) + t * 32 + r32;
            f.a[kb][t] = *reinterpret_cast<const V*>(la + ra * ROWB + swz(ra, C0 + 2 * kb + h) * 16);
        }
#pragma unroll
        for (int t = 0; t < WNT; t++) f.b[kb][t] = read_b_nn16<BN, HALF, V>(lb, wn * (WNT * 32) + t * 32, kb, lane);
    }
}

// 16-bit fragments with either operand given transposed: A M-major (A as [K, M], M contiguous:
// the vjp's g^T operand) takes the same slot layout and transposing reads as N-major B, with BM
// for BN.
template <int DT, int TM, int WNT, int BM, int BN, int HALF, bool AT, bool BT>
__device__ __forceinline__ void read_frags_t16(Frags<DT, TM, WNT>& f, const char* la, const char* lb, int wm, int wn,
                                               int lane) {
    using V = std::remove_reference_t<decltype(f.b[0][0])>;
    const int r32 = lane & 31, h = lane >> 5;
    constexpr int C0 = HALF * STEP_CHUNKS;
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
#pragma unroll
        for (int t = 0; t < TM; t++) {
            const int ra = wm * (TM * 32) + t * 32 + r32;
            if constexpr (AT) f.a[kb][t] = read_b_nn16<BM, HALF, V>(la, wm * (TM * 32) + t * 32, kb, lane);
            else f.a[kb][t] = *reinterpret_cast<const V*>(la + ra * ROWB + swz(ra, C0 + 2 * kb + h) * 16);
        }
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int rb = wn * (WNT * 32) + t * 32 + r32;
            if constexpr (BT) f.b[kb][t] = read_b_nn16<BN, HALF, V>(lb, wn * (WNT * 32) + t * 32, kb, lane);
            else f.b[kb][t] = *reinterpret_cast<const V*>(lb + rb * ROWB + swz(rb, C0 + 2 * kb + h) * 16);
        }
    }
}

// DMA of the 16-bit N-major B slot: one instruction fills 1 KB = 512 / BN K rows; wave w's
// instruction i fills rows RPI (N w + i) ..; lane L lands at row RPI (N w + i) + L / (BN / 8),
// stored chunk L % (BN / 8), so it fetches the logical chunk swz_nn16 stores there.  Columns past
// N load the row's last whole chunk (N is a multiple of 8; those C columns are never stored).
template <int BN, int N>
__device__ __forceinline__ DmaOffsets<N> dma_offsets_nn16(uint32_t cols_valid, uint32_t ldk, int wave, int lane) {
    constexpr int CPRN = BN / 8;                         // 16-byte chunks per K row
    constexpr int RPI = 64 / CPRN;                       // K rows per DMA instruction
    DmaOffsets<N> o;
#pragma unroll
    for (int i = 0; i < N; i++) {
        const int row = (wave * N + i) * RPI + lane / CPRN;
        const uint32_t col = min((uint32_t)swz_nn16(row, lane % CPRN) * 8, cols_valid - 8);
        o.v[i] = ((uint32_t)row * ldk + col) * 2u;
    }
    return o;
}

// One K step (32 rows) of the 16-bit N-major B tile through registers, element loads, zero past K
// and past N, into rows 0 .. 31 of the slot.  Thread chunk q = tid + 256 j is K row q / (BN / 8),
// logical chunk q % (BN / 8).
template <int BN, int NT = NTHREADS> constexpr int kTailChunksNN16 = 32 * (BN / 8) / NT;

template <int BN, int NT = NTHREADS>
__device__ __forceinline__ void load_tile_guarded_nn16(uint4 (&r)[(kTailChunksNN16<BN, NT>)],
                                                       const uint16_t* __restrict__ base, uint32_t cols_valid,
                                                       uint32_t ldk, uint32_t k0, uint32_t K) {
#pragma unroll
    for (int j = 0; j < kTailChunksNN16<BN, NT>; j++) {
        const int q = threadIdx.x + NT * j;
        const uint32_t k = k0 + (uint32_t)(q / (BN / 8));
        const uint32_t c = (uint32_t)(q % (BN / 8)) * 8;
        uint16_t tmp[8];
#pragma unroll
        for (int e = 0; e < 8; e++) tmp[e] = (k < K && c + e < cols_valid) ? base[(uint64_t)k * ldk + c + e] : 0;
        __builtin_memcpy(&r[j], tmp, 16);
    }
}

template <int BN, int NT = NTHREADS>
__device__ __forceinline__ void store_tile_nn16(char* lds, const uint4 (&r)[(kTailChunksNN16<BN, NT>)]) {
#pragma unroll
    for (int j = 0; j < kTailChunksNN16<BN, NT>; j++) {
        const int q = threadIdx.x + NT * j;
        const int row = q / (BN / 8), c = q % (BN / 8);
        *reinterpret_cast<uint4*>(lds + row * (BN * 2) + swz_nn16(row, c) * 16) = r[j];
    }
}

// s_waitcnt vmcnt(N), expcnt / lgkmcnt left at their maximum (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmem() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Instruction order within a K step, so the LDS and the memory pipeline work under the matrix
// core instead of before it (sched_group_barrier masks: 0x008 MFMA, 0x100 LDS read, 0x020
// vector-memory read).  A slot is one MFMA for 16-bit types and four for fp32; a step has
// 2 TM WNT slots, 2 (TM + WNT) fragment reads, and a pair's ND DMA instructions per wave.  The fragment reads go out early in their window so that they have returned (LDS
// latency is several MFMAs) before the next step's first MFMA needs them.
template <int DT> constexpr int kMfmaPerSlot = DT == MX_FLOAT32 ? 4 : 1;

// First step of a pair: the next step's fragment reads, one after each leading MFMA slot.  The
// pair's first MFMA goes before the first read: LDS reads complete in order, so an MFMA behind a
// new read would wait for that read as well as for its own (long since loaded) fragments.
template <int DT, int TM, int WNT, int NR>
__device__ __forceinline__ void interleave_even() {
    constexpr int MF = kMfmaPerSlot<DT>, SLOTS = 2 * TM * WNT;
    constexpr int RPS = (NR + SLOTS - 1) / SLOTS;              // reads per slot
    constexpr int USED = (NR + RPS - 1) / RPS;                 // slots that carry reads
    static_assert(USED <= SLOTS, "interleave counts");
#pragma unroll
    for (int i = 0; i < USED; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, RPS, 0);
    }
    if constexpr (SLOTS > USED) __builtin_amdgcn_sched_group_barrier(0x008, (SLOTS - USED) * MF, 0);
}

// Second step of a pair, after its barrier (TM WNT slots left): the next step's fragment reads
// over the first half of the slots, the DMA of the pair two ahead over all of them.
template <int DT, int TM, int WNT, int ND, int NR>
__device__ __forceinline__ void interleave_odd() {
    constexpr int MF = kMfmaPerSlot<DT>, H = TM * WNT;
    constexpr int RPS = NR / (H / 2);                          // reads per slot, first half
    constexpr int D1 = (ND + H - 1) / H;                       // DMAs per slot, first half
    constexpr int D2 = (ND - D1 * (H / 2)) / (H / 2);          // DMAs per slot, second half
    static_assert(RPS * (H / 2) == NR && D1 * (H / 2) + D2 * (H / 2) == ND, "interleave counts");
#pragma unroll
    for (int i = 0; i < H / 2; i++) {
        __builtin_amdgcn_sched_group_barrier(0x100, RPS, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, D1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
    }
#pragma unroll
    for (int i = 0; i < H / 2; i++) {
        if constexpr (D2 > 0) __builtin_amdgcn_sched_group_barrier(0x020, D2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
    }
}

// Workgroup barrier for the DMA ring.  __syncthreads() carries a workgroup release fence that
// waits for every outstanding vector-memory operation.  The ring orders its LDS traffic itself:
// each wave waits (vmcnt) for its DMA of the pair it is about to read, and a slot is refilled
// only after the barrier that follows every wave's reads of it (lgkmcnt(0): this wave's reads
// have returned).  The wait is the compiler's own s_waitcnt (lgkmcnt(0); vmcnt / expcnt at their
// maximum), so its wait bookkeeping knows every fragment read has returned; s_barrier needs no
// implicit wait on gfx950 (back-off barrier), and the empty asm statements keep LDS accesses from
// moving across.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The epilogue of the K-major / 16-bit tile kernels: acc[i][j][4 q + e] is C[row, col] with
// row = 32 i + lane % 32 and col = 32 j + 8 q + 4 (lane / 32) + e (the C^T fragment, see mma_step)
// of the wave's (wm, wn) quarter of the tile at (m0, n0).
// An interior tile with unit-stride 16-byte aligned C rows goes through LDS when the wave's quarter
// fits `stage` (STAGE: 16-bit results, and fp32 128 x 128 tiles): the fragment layout would make
// every store instruction touch 32 rows with 16 bytes each (a 256 x 2048 x 64 f16 product, one K
// pair, took 19 us for its 32 MB of C); staged, 64 lanes store whole 16-byte chunks of consecutive
// row bytes.  The quarter is written to LDS whole (16-byte chunk c of row r at
// c ^ (r mod chunks per row)), then read back and stored row-major.  Otherwise an interior tile
// stores 4 columns per instruction from the fragments, and other tiles one element at a time.
template <int DT, int BM, int BN, int WN, bool SPLIT, class Src, bool STAGE, typename CT, bool RT = false>
__device__ __forceinline__ void store_c(CT* Cbat, const f16v (&acc)[BM / 64][BN / (32 * WN)], const GemmArgs& g,
                                        const typename Src::Geom& geo, uint32_t m0, uint32_t n0, int wm, int wn, int lane,
                                        bool vec_store, char* stage) {
    constexpr int TM = BM / 64, WNT = BN / (32 * WN);
    const int h = lane >> 5, c32 = lane & 31;
    // row of accumulator tile i within the wave's range (RT: fp32 M-major A, Frags32T)
    auto rin = [&](int i) { return RT ? TM * c32 + i : i * 32 + c32; };
    auto cvt = [](float v) -> CT {
        if constexpr (SPLIT || DT == MX_FLOAT32) return v;
        else if constexpr (DT == MX_FLOAT16) return float_to_half_bits(v);
        else return float_to_bf16(v);
    };
    const bool interior = m0 + BM <= g.M && n0 + BN <= g.N && vec_store;
    if constexpr (STAGE) {
        if (interior) {
            constexpr int RB = WNT * 32 * (int)sizeof(CT);       // bytes of a staged row
            constexpr int CPRS = RB / 16;                        // 16-byte chunks per staged row
            constexpr int EPC = 16 / (int)sizeof(CT);            // elements per chunk
            static_assert((CPRS & (CPRS - 1)) == 0 && CPRS <= 32, "staged row chunks");
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int r = rin(i);
#pragma unroll
                for (int j = 0; j < WNT; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int col = j * 32 + 8 * q + 4 * h;
                        char* dst = stage + r * RB + (((col / EPC) ^ (r & (CPRS - 1))) * 16) + (col % EPC) * (int)sizeof(CT);
                        if constexpr (sizeof(CT) == 4) {
                            *reinterpret_cast<f4v*>(dst) = f4v{acc[i][j][4 * q], acc[i][j][4 * q + 1],
                                                               acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                        } else {
                            uint2 v;
                            v.x = (uint32_t)cvt(acc[i][j][4 * q]) | ((uint32_t)cvt(acc[i][j][4 * q + 1]) << 16);
                            v.y = (uint32_t)cvt(acc[i][j][4 * q + 2]) | ((uint32_t)cvt(acc[i][j][4 * q + 3]) << 16);
                            *reinterpret_cast<uint2*>(dst) = v;
                        }
                    }
            }
            // LDS accesses of one wave complete in order: the reads below see the writes above
            __builtin_amdgcn_s_waitcnt(0xC07F);
            asm volatile("" ::: "memory");
            const uint32_t row0 = m0 + wm * (TM * 32);
            CT* cbase = Cbat + n0 + wn * (WNT * 32);
            constexpr int RPI = 64 / CPRS;                       // rows per store instruction
            const int c = lane % CPRS;
            // streaming stores: C is not read again here, and kept out of the L2 it leaves room
            // for the operands (f16 3x3 convolution 24.9 -> 23.7 us, the f16 GEMM with B
            // N-major 1091 -> 1133 TFLOP/s); split partials, which the sum reads next, stay cached
            typedef unsigned u4v __attribute__((ext_vector_type(4)));
#pragma unroll 8
            for (int it = 0; it < TM * 32 / RPI; it++) {
                const int rr = it * RPI + lane / CPRS;
                const u4v v = *reinterpret_cast<const u4v*>(stage + rr * RB + ((c ^ (rr & (CPRS - 1))) * 16));
                u4v* dst = reinterpret_cast<u4v*>(cbase + Src::row_off(g, geo, row0 + rr) + c * EPC);
                if constexpr (SPLIT) *dst = v;                   // partials: read back next
                else __builtin_nontemporal_store(v, dst);
            }
            return;
        }
    }
    if (interior) {                                           // 4 columns per store
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const uint32_t row = m0 + wm * (TM * 32) + rin(i);
            CT* crow = Cbat + Src::row_off(g, geo, row) + n0 + wn * (WNT * 32) + 4 * h;
#pragma unroll
            for (int j = 0; j < WNT; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    CT* p = crow + j * 32 + 8 * q;
                    if constexpr (sizeof(CT) == 4) {
                        *reinterpret_cast<float4*>(p) =
                            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
                    } else {
                        uint2 v;
                        v.x = (uint32_t)cvt(acc[i][j][4 * q]) | ((uint32_t)cvt(acc[i][j][4 * q + 1]) << 16);
                        v.y = (uint32_t)cvt(acc[i][j][4 * q + 2]) | ((uint32_t)cvt(acc[i][j][4 * q + 3]) << 16);
                        *reinterpret_cast<uint2*>(p) = v;
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const uint32_t row = m0 + wm * (TM * 32) + rin(i);
        if (row >= g.M) continue;
        CT* crow = Cbat + Src::row_off(g, geo, row);
#pragma unroll
        for (int j = 0; j < WNT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t col = n0 + wn * (WNT * 32) + j * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                if (col < g.N) crow[(uint64_t)col * g.cn] = cvt(acc[i][j][r]);
            }
    }
}

// ------------------------------------------------------------------ the tile kernel
// Src provides:
//   Geom                                  extra kernel argument (empty for GEMM)
//   static constexpr bool kStrided        A may take the guarded K-tail path
//   AState a_init<S, NA>(g, geo, m0, rows_a, wave, lane)    per-lane A addressing state
//   void a_dma<S, NA>(lds, A, st, g, geo, m0, pair, wave, lane)   one pair of the A slot
//   uint64_t row_off(g, geo, row)         element offset of C row `row` (batch offset apart)
//   bool row_vec_ok<S>(g, geo)            every row offset is a multiple of 16 bytes
// (NA = DMA instructions per wave for the A slot.)  Tiles are BM x BN with BM, BN in {128, 256}:
// 2 x WN waves of (BM / 2) x (BN / WN).  A 128 x 128 tile needs 64 KB of LDS, so two blocks share
// a CU.
// SPLIT: the K range is cut into g.ksplit-element pieces, one per block along the outermost
// block-batch index; the block writes its fp32 partial tile to Cv as [split][batch][M][N]
// (g.ldc = N, g.cn = 1), and a second kernel sums the splits in order.
// BNN: Bt is N-major (B as [K, N]: g.ldb == 1, g.kb is B's row stride); fp32 reads it as FragsNN
// describes, 16-bit types through transposing LDS reads (read_frags_nn16).
template <int DT, int BM, int BN, bool VEC, bool SPLIT, class Src, bool BNN = false, bool AMN = false, int WN = 2>
__global__ __launch_bounds__(128 * WN) void mfma_tile_kernel(void* __restrict__ Cv,
                                                             const typename MmaTraits<DT>::S* __restrict__ A,
                                                             const typename MmaTraits<DT>::S* __restrict__ Bt,
                                                             GemmArgs g, typename Src::Geom geo) {
    using S = typename MmaTraits<DT>::S;
    using CT = std::conditional_t<SPLIT, float, S>;    // element type written to Cv
    static_assert(WN == 2 || (WN == 4 && (DT != MX_FLOAT32 || !AMN)), "eight waves");
    constexpr int NW = 2 * WN, NT = 64 * NW;           // waves (2 along M, WN along N), threads
    constexpr int TM = BM / 64;                        // A tiles of 32 rows per wave
    constexpr int WNT = BN / (32 * WN);                // Bt tiles of 32 rows per wave
    constexpr int KSTEP = STEPB / sizeof(S);           // elements of K per step
    constexpr int SLOT_A = BM * ROWB, SLOT_B = BN * ROWB;
    constexpr int DMA_A = kDma<BM, NW>, DMA_B = kDma<BN, NW>;
    // two pair slots per operand, each its own array so the compiler tells the DMA into one
    // slot from the fragment reads of the other
    __shared__ __align__(16) char la0[SLOT_A], la1[SLOT_A];
    __shared__ __align__(16) char lb0[SLOT_B], lb1[SLOT_B];
    auto slot_a = [&](auto s) -> char* {
        if constexpr (decltype(s)::value == 0) return la0;
        else return la1;
    };
    auto slot_b = [&](auto s) -> char* {
        if constexpr (decltype(s)::value == 0) return lb0;
        else return lb1;
    };

    uint32_t bidx, tm, tn;
    tile_of(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n, bidx, tm, tn);
    uint64_t offA = 0, offB = 0, offC = 0;                // batch offsets
    uint32_t Klen = g.K;                                  // this block's K range: kbeg .. + Klen
    if constexpr (SPLIT) {
        const uint32_t split = bidx / g.batches;
        bidx -= split * g.batches;
        const uint32_t kbeg = split * g.ksplit;
        Klen = g.K - kbeg < g.ksplit ? g.K - kbeg : g.ksplit;
        offA = (uint64_t)kbeg * g.ka;
        offB = (uint64_t)kbeg * g.kb;
        offC = ((uint64_t)split * g.batches + bidx) * g.M * g.N;
    }
    {
        uint32_t rem = bidx;
        for (int d = g.bd.n - 1; d >= 0; --d) {
            uint32_t q = g.bd.shape[d].div(rem);
            uint32_t idx = rem - q * g.bd.shape[d].d;
            rem = q;
            offA += (uint64_t)idx * g.bd.sA[d];
            offB += (uint64_t)idx * g.bd.sB[d];
            if constexpr (!SPLIT) offC += (uint64_t)idx * g.bd.sC[d];
        }
    }
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const S* Abat = A + offA;
    const S* Bblk = Bt + offB + (uint64_t)n0 * g.ldb;
    const uint32_t rows_a = g.M - m0 < (uint32_t)BM ? g.M - m0 : (uint32_t)BM;
    const uint32_t rows_b = g.N - n0 < (uint32_t)BN ? g.N - n0 : (uint32_t)BN;

    // the wave index is wave-uniform: keeping it in a scalar register keeps every LDS slot
    // address derived from it (the DMA destinations) scalar too
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;

    constexpr bool NN32 = BNN && DT == MX_FLOAT32;      // fp32 N-major B (FragsNN)
    constexpr bool NN16 = BNN && DT != MX_FLOAT32;      // 16-bit N-major B (transposing reads)
    static_assert(!AMN || Src::kStrided, "M-major A: matrices only");
    constexpr bool T32 = AMN && DT == MX_FLOAT32;        // fp32 M-major A (Frags32T, rows remapped)
    f16v acc[TM][WNT];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < WNT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const uint32_t KT = (Klen + KSTEP - 1) / KSTEP;
    const uint32_t KP = VEC ? Klen / (2 * KSTEP) : 0;  // whole K pairs copied by LDS DMA
    // Fragments are double-buffered in registers: f0 holds a pair's first step, f1 its second;
    // each step reads the next step's fragments while its own MFMAs run.
    using FR = std::conditional_t<T32, Frags32T<TM, WNT, BNN>,
                                  std::conditional_t<NN32, FragsNN<TM, WNT>, Frags<DT, TM, WNT>>>;
    FR f0, f1;
    auto read_step = [&](auto half, FR& f, const char* la, const char* lb) {
        constexpr int HALF = decltype(half)::value;
        if constexpr (T32) read_frags_32t<TM, WNT, BM, BN, HALF, BNN>(f, la, lb, wm, wn, lane);
        else if constexpr (NN32) read_frags_nn<TM, WNT, BN, HALF>(f, la, lb, wm, wn, lane);
        else if constexpr (AMN) read_frags_t16<DT, TM, WNT, BM, BN, HALF, true, NN16>(f, la, lb, wm, wn, lane);
        else if constexpr (NN16) read_frags_nn16<DT, TM, WNT, BN, HALF>(f, la, lb, wm, wn, lane);
        else read_frags<DT, TM, WNT, HALF>(f, la, lb, wm, wn, lane);
    };
    auto mma = [&](auto i0, auto i1, const FR& f) {
        constexpr int I0_ = decltype(i0)::value, I1_ = decltype(i1)::value;
        if constexpr (T32) mma_step_32t<TM, WNT, I0_, I1_, BNN>(acc, f);
        else if constexpr (NN32) mma_step_nn<TM, WNT, I0_, I1_>(acc, f);
        else mma_step<DT, TM, WNT, I0_, I1_>(acc, f);
    };
    // LDS reads per step: one 16-byte read per A fragment and per K-major B fragment, two 8-byte
    // transposing reads per N-major one
    constexpr int NREADS = 2 * ((AMN ? 2 : 1) * TM + (NN16 ? 2 : 1) * WNT);
    const auto sa = Src::template a_init<S, DMA_A>(g, geo, m0, rows_a, wave, lane);
    // M-major A: the slot's K rows of BM elements, from the tile's first column
    const DmaOffsets<DMA_A> oa_mn = !AMN ? DmaOffsets<DMA_A>{}
                                    : T32 ? dma_offsets_nn<BM, DMA_A>(rows_a, g.ka, wave, lane)
                                          : dma_offsets_nn16<BM, DMA_A>(rows_a, g.ka, wave, lane);
    const S* Amn = Abat + m0;
    const DmaOffsets<DMA_B> ob = NN32   ? dma_offsets_nn<BN, DMA_B>(rows_b, g.kb, wave, lane)
                                 : NN16 ? dma_offsets_nn16<BN, DMA_B>(rows_b, g.kb, wave, lane)
                                        : dma_offsets<S, DMA_B>(rows_b, g.ldb, wave, lane);
    auto dma_pair = [&](auto s, uint32_t p) {
        if constexpr (AMN) dma_rows<S, DMA_A>(slot_a(s), Amn + (uint64_t)p * 2 * KSTEP * g.ka, oa_mn, 0, wave);
        else Src::template a_dma<S, DMA_A>(slot_a(s), Abat, sa, g, geo, m0, p, wave, lane);
        if constexpr (BNN) dma_rows<S, DMA_B>(slot_b(s), Bblk + (uint64_t)p * 2 * KSTEP * g.kb, ob, 0, wave);
        else dma_rows<S, DMA_B>(slot_b(s), Bblk, ob, p * 2 * KSTEP, wave);
    };
    constexpr int H0 = TM / 2;                           // A tile rows of a step's first half
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using IH = std::integral_constant<int, H0>;
    using ITM = std::integral_constant<int, TM>;
    constexpr int PER_PAIR = DMA_A + DMA_B;              // DMA instructions per wave per pair
    // Pair p lives in slot p % 2.  Its first step reads the second step's fragments (same slot,
    // already landed) while the first step's MFMAs run; no barrier.  Its second step runs half of
    // its MFMAs, waits for pair p + 1's DMA (the only one in flight), and meets the barrier --
    // after which every wave has read all of pair p's fragments -- then refills slot p % 2 with
    // pair p + 2 and reads pair p + 1's first fragments under the remaining MFMAs.  Steady pairs
    // have no branches, so the compiler's own wait bookkeeping stays exact; sched_barrier(0)
    // fences keep each phase's instructions inside it.
    // fp32 takes no interleave groups: with four MFMAs per slot the scheduler filled each group
    // with four MFMAs on one accumulator (a dependent chain); left alone it alternates the 16
    // accumulators.  It also reads the next pair's first fragments before issuing the DMA, since
    // the compiler otherwise makes the reads after the DMA wait for it.  (fp32 main GEMM: 118 ->
    // 127 TFLOP/s.)
    auto pair_steady = [&](auto s, uint32_t p) {
        using SN = std::integral_constant<int, 1 - decltype(s)::value>;
        constexpr int MF = kMfmaPerSlot<DT>;
        // a wave between barriers runs its MFMAs at raised priority, ahead of a wave on the same
        // SIMD that is issuing its DMA and fragment reads after the barrier (f16 GEMM +2%)
        __builtin_amdgcn_s_setprio(1);
        read_step(I1{}, f1, slot_a(s), slot_b(s));
        mma(I0{}, ITM{}, f0);
        if constexpr (DT != MX_FLOAT32) interleave_even<DT, TM, WNT, NREADS>();
        __builtin_amdgcn_sched_barrier(0);
        mma(I0{}, IH{}, f1);
        if constexpr (DT != MX_FLOAT32) __builtin_amdgcn_sched_group_barrier(0x008, TM * WNT * MF, 0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        wait_vmem<0>();
        ring_barrier();
        if constexpr (DT == MX_FLOAT32) {
            // fp32: the next pair's first fragments before the DMA, so no LDS read follows it
            read_step(I0{}, f0, slot_a(SN{}), slot_b(SN{}));
            dma_pair(s, p + 2);
        } else {
            dma_pair(s, p + 2);
            read_step(I0{}, f0, slot_a(SN{}), slot_b(SN{}));
        }
        mma(IH{}, ITM{}, f1);
        if constexpr (DT != MX_FLOAT32) interleave_odd<DT, TM, WNT, PER_PAIR, NREADS>();
        __builtin_amdgcn_sched_barrier(0);
    };
    // the last pairs: no DMA past the end, no barrier after the last
    auto pair_drain = [&](auto s, uint32_t p) {
        using SN = std::integral_constant<int, 1 - decltype(s)::value>;
        if (p >= KP) return;
        read_step(I1{}, f1, slot_a(s), slot_b(s));
        mma(I0{}, ITM{}, f0);
        mma(I0{}, IH{}, f1);
        // (the MFMA sequence is the same on both paths: a branch around MFMAs makes the
        // compiler shuffle the accumulators between register files)
        if (p + 1 < KP) {
            wait_vmem<0>();
            ring_barrier();
            if (p + 2 < KP) dma_pair(s, p + 2);
            read_step(I0{}, f0, slot_a(SN{}), slot_b(SN{}));
        }
        mma(IH{}, ITM{}, f1);
    };
    if (KP > 0) {
        dma_pair(I0{}, 0);
        if (KP > 1) {
            dma_pair(I1{}, 1);
            wait_vmem<PER_PAIR>();
        } else {
            wait_vmem<0>();
        }
        ring_barrier();
        read_step(I0{}, f0, la0, lb0);
        uint32_t p = 0;
        for (; p + 4 <= KP; p += 2) {                    // pairs p, p + 1 issue p + 2, p + 3
            pair_steady(I0{}, p);
            pair_steady(I1{}, p + 1);
        }
        // p is even here; at most 3 pairs remain
        pair_drain(I0{}, p);
        pair_drain(I1{}, p + 1);
        pair_drain(I0{}, p + 2);
        __syncthreads();                                  // every wave is done with the slots
    }
    if constexpr (Src::kStrided) {
        // K tail (and every step of strided operands): element loads through registers into the
        // first half of slot 0, zero past K.
        const S* Ablk = Abat + (uint64_t)m0 * g.lda;
        for (uint32_t kt = 2 * KP; kt < KT; kt++) {
            if constexpr (T32) {
                f4v ra[kTailChunksNN<BM, NT>];
                load_tile_guarded_nn<BM, NT>(ra, reinterpret_cast<const float*>(Amn), rows_a, g.ka, kt * KSTEP, Klen);
                store_tile_nn<BM, NT>(la0, ra);
            } else if constexpr (AMN) {
                uint4 ra[kTailChunksNN16<BM, NT>];
                load_tile_guarded_nn16<BM, NT>(ra, reinterpret_cast<const uint16_t*>(Amn), rows_a, g.ka, kt * KSTEP, Klen);
                store_tile_nn16<BM, NT>(la0, ra);
            } else {
                uint4 ra[kTailChunks<BM, NT>];
                load_tile_guarded<S, BM, NT>(ra, Ablk, rows_a, g.lda, g.ka, kt * KSTEP, Klen);
                store_tile<BM, NT>(la0, ra);
            }
            if constexpr (NN32) {
                f4v rb[kTailChunksNN<BN, NT>];
                load_tile_guarded_nn<BN, NT>(rb, reinterpret_cast<const float*>(Bblk), rows_b, g.kb, kt * KSTEP, Klen);
                store_tile_nn<BN, NT>(lb0, rb);
            } else if constexpr (NN16) {
                uint4 rb[kTailChunksNN16<BN, NT>];
                load_tile_guarded_nn16<BN, NT>(rb, Bblk, rows_b, g.kb, kt * KSTEP, Klen);
                store_tile_nn16<BN, NT>(lb0, rb);
            } else {
                uint4 rb[kTailChunks<BN, NT>];
                load_tile_guarded<S, BN, NT>(rb, Bblk, rows_b, g.ldb, g.kb, kt * KSTEP, Klen);
                store_tile<BN, NT>(lb0, rb);
            }
            __syncthreads();
            read_step(I0{}, f0, la0, lb0);
            mma(I0{}, ITM{}, f0);
            __syncthreads();
        }
    }

    // epilogue: acc[i][j][4 q + e] is C[row, col] with row = 32 i + lane % 32 (fp32 M-major A:
    // TM (lane % 32) + i) and col = 32 j + 8 q + 4 (lane / 32) + e (the C^T fragment, see mma_step)
    CT* Cbat = static_cast<CT*>(Cv) + offC;
    const int h = lane >> 5, c32 = lane & 31;
    const bool vec_store = g.cn == 1 && Src::template row_vec_ok<CT>(g, geo) && ((uintptr_t)Cbat % 16) == 0;
    if constexpr (NN32) {
        // accumulator q of MFMA tile (i, .) holds, in register r, C column
        // WNT (8 (r / 4) + 4 h + r % 4) + q of the wave's column range
        const uint32_t cw = n0 + wn * (WNT * 32);
        typedef float cvec __attribute__((ext_vector_type(WNT)));
        const bool interior = m0 + BM <= g.M && n0 + BN <= g.N && vec_store;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const uint32_t row = m0 + wm * (TM * 32) + (T32 ? TM * c32 + i : i * 32 + c32);
            if (!interior && row >= g.M) continue;
            CT* crow = Cbat + Src::row_off(g, geo, row);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t col = cw + WNT * (8 * (r >> 2) + 4 * h + (r & 3));
                if (interior) {
                    cvec v;
#pragma unroll
                    for (int q = 0; q < WNT; q++) v[q] = acc[i][q][r];
                    *reinterpret_cast<cvec*>(crow + col) = v;
                } else {
#pragma unroll
                    for (int q = 0; q < WNT; q++)
                        if (col + q < g.N) crow[(uint64_t)(col + q) * g.cn] = acc[i][q][r];
                }
            }
        }
        return;
    }
    // the epilogue's LDS stage: this wave's part of C (NW / 4 waves per slot array) in one of the
    // four slot arrays (free now: every wave has passed the barrier after its last fragment reads)
    constexpr int QB = (BM / 2) * (BN / WN) * (int)sizeof(CT), WPS = NW / 4;
    constexpr bool STAGE = QB * WPS <= (SLOT_A < SLOT_B ? SLOT_A : SLOT_B);
    const int sw = wave / WPS;
    char* stage = (sw == 0 ? la0 : sw == 1 ? la1 : sw == 2 ? lb0 : lb1) + (wave % WPS) * QB;
    store_c<DT, BM, BN, WN, SPLIT, Src, STAGE, CT, T32>(Cbat, acc, g, geo, m0, n0, wm, wn, lane, vec_store, stage);
}

// Tile shape for a problem: 256 x 256 tiles while they give at least one block per CU (256), 256 x
// 128 (N <= 128) while they give two (512); otherwise 128 x 128 tiles, two blocks per CU.
// Measured: 4096 x 4096 x 512 on 256 x 256 tiles fp32 113-126 / f16 539 TFLOP/s, on 128 x 128
// 101-107 / 510; the f16 3 x 3 convolution's 392 tiles of 256 x 128 ran 34.7 us against 32.2 us
// on 128 x 128.
struct TileShape { int bm, bn; };

// 16-bit tiles and fp32 tiles with A K-major (256 x 256 and 128 x 128) run eight waves (2 x 4:
// 128 x 64 / 64 x 32 each), twice the waves per SIMD, so one wave's MFMAs cover another's waits,
// against 1.5x the fragment reads (fp32: config 3's product 136 -> 146-147 TFLOP/s, with B
// N-major 134 -> 144, the 256 x 256 tile no longer spilling; the 3x3 convolution 157 -> 154 us; the
// MLP step 0.606-0.616 -> 0.601 ms).  fp32 with A M-major keeps four.
// Config 3's f16 product: 1001-1008 -> 1026-1034 TFLOP/s in one process, B read N-major
// 1043-1047 -> 1085; config 4's f16 3x3 convolution 26.5 -> 25.5 us, 1x1 stride 2 12.8 -> 12.2 us.
// (256 x 256 convolution tiles keep four: the gather's per-lane state would spill.)
constexpr bool kWide16 = true;
inline TileShape choose_tile(uint64_t M, uint64_t N, uint64_t batches) {
    const int bn = N <= 128 ? 128 : 256;
    const uint64_t big = (M + 255) / 256 * ((N + bn - 1) / bn) * batches;
    if (big >= (bn == 256 ? 256u : 512u)) return {256, bn};
    return {128, 128};
}

// Launches mfma_tile_kernel<DT, BM, BN, VEC, SPLIT, Src> for the chosen shape; with SPLIT,
// nsplit K pieces of g.ksplit elements each.
template <int DT, bool VEC, bool SPLIT, class Src, bool BNN = false, bool AMN = false>
int launch_tile_kernel(TileShape ts, GemmArgs g, typename Src::Geom geo, void* C, const void* A, const void* Bt,
                       hipStream_t st, const char* who, uint32_t nsplit = 1) {
    using S = typename MmaTraits<DT>::S;
    auto go = [&](auto bm, auto bn, auto wn) -> int {
        constexpr int BM = decltype(bm)::value, BN = decltype(bn)::value, WN = decltype(wn)::value;
        g.tiles_m = (g.M + BM - 1) / BM;
        g.tiles_n = (g.N + BN - 1) / BN;
        const uint64_t blocks = (uint64_t)g.tiles_m * g.tiles_n * g.batches * nsplit;
        if (blocks > 0x7fffffffull) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": grid too large");
        hipLaunchKernelGGL((mfma_tile_kernel<DT, BM, BN, VEC, SPLIT, Src, BNN, AMN, WN>), dim3((uint32_t)blocks),
                           dim3(128 * WN), 0, st, C, (const S*)A, (const S*)Bt, g, geo);
        MX_HIP(hipGetLastError());
        return MX_OK;
    };
    using I2 = std::integral_constant<int, 2>;
    using I128 = std::integral_constant<int, 128>;
    using I256 = std::integral_constant<int, 256>;
    if (ts.bm == 256 && ts.bn == 256) {
        if constexpr ((DT != MX_FLOAT32 || !AMN) && Src::kStrided)  // (conv: the gather's state would spill)
            if (kWide16) return go(I256{}, I256{}, std::integral_constant<int, 4>{});
        return go(I256{}, I256{}, I2{});
    }
    if (ts.bm == 256) return go(I256{}, I128{}, I2{});
    if constexpr (DT != MX_FLOAT32 || (!BNN && !AMN))
        if (kWide16) return go(I128{}, I128{}, std::integral_constant<int, 4>{});
    return go(I128{}, I128{}, I2{});
}

// A strided matrix operand (batched MatMul).
struct MatrixSrc {
    struct Geom {};
    static constexpr bool kStrided = true;
    template <typename S, int NA>
    __device__ __forceinline__ static DmaOffsets<NA> a_init(const GemmArgs& g, const Geom&, uint32_t m0,
                                                            uint32_t rows_a, int wave, int lane) {
        return dma_offsets<S, NA>(rows_a, g.lda, wave, lane);
    }
    template <typename S, int NA>
    __device__ __forceinline__ static void a_dma(char* lds, const S* Abat, const DmaOffsets<NA>& o,
                                                 const GemmArgs& g, const Geom&, uint32_t m0, uint32_t p, int wave,
                                                 int lane) {
        constexpr int KSTEP = STEPB / sizeof(S);
        dma_rows<S, NA>(lds, Abat + (uint64_t)m0 * g.lda, o, p * 2 * KSTEP, wave);
    }
    __device__ __forceinline__ static uint64_t row_off(const GemmArgs& g, const Geom&, uint32_t row) {
        return (uint64_t)row * g.ldc;
    }
    template <typename S>
    __device__ __forceinline__ static bool row_vec_ok(const GemmArgs& g, const Geom&) {
        return ((uint64_t)g.ldc * sizeof(S)) % 16 == 0;
    }
};

}  // namespace tile
}  // namespace mx
