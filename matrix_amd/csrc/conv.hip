// conv.hip -- ConvolutionND, channels-last, as an implicit GEMM on the matrix cores.
//
// Replaces conv_gpu / conv2d_gpu (Matrix.mm:12335-12395, Matrix.mm:5521-5559) and their Metal
// kernels (ConvolutionND.metal:18-372).  The semantics are those of the reference's CPU conv
// (conv_cpu, Matrix.mm:12397-12500 == conv2d_cpu, Matrix.mm:5668-5741): input [N, S1..Sn, C],
// kernel [O, K1..Kn, C / groups], output [N, O1..On, O], each with arbitrary element strides;
// output position o samples input position o * stride - pad_lo + k * dil_rhs of the input
// dilated by dil_lhs (taps off the image or between dilated samples contribute nothing); output
// channel oc uses input channels of group oc / (O / groups); flip reads the kernel back to
// front.  The reduction runs over (kernel position, channel), channel fastest.
//
// float32 / float16 / bfloat16, 1 or 2 spatial axes, no input dilation: implicit GEMM.
//   C[m, o] = sum_k A[m, k] Wp[o, k] with m = (n, o1.., on) and k = (kernel position, channel).
//   The image is packed (when it is not already so) into channels-last Xp [N, S.., groups, Cgp]
//   and the kernel into Wp [O, K.., Cgp], Cgp = C / groups rounded up to a 128-byte K pair with
//   zero channels, flip applied.  Every K pair then lies inside one kernel position, so the A
//   tile's DMA gathers whole 128-byte channel runs straight from Xp: one address per lane per
//   DMA instruction, zeros for taps outside the image (an offset past the buffer resource's
//   range).  Groups are the GEMM batch.
// Everything else (integers, input dilation, 3+ spatial axes): a direct kernel, one output per
//   thread, in the reference's loop order (fp32 results then equal the CPU's bit for bit).
#include "mfma_tile.hpp"

namespace mx {
namespace {

using tile::GemmArgs;
using tile::MmaTraits;

constexpr int kMaxSpatial = 6;

// ------------------------------------------------------------------ implicit-GEMM A operand
template <int NS>
struct ConvSrc {
    struct Geom {
        FastDiv odim[NS];        // output spatial extents, outermost first
        uint32_t idim[NS];       // input spatial extents
        int32_t stride[NS], dil[NS], pad[NS];
        FastDiv kdim[NS];        // kernel spatial extents
        uint32_t xs[NS];         // Xp element stride of each spatial axis
        uint32_t xn;             // Xp element stride of N
        FastDiv cpairs;          // K pairs per kernel position (Cgp / pair elements)
        uint32_t on, os[NS];     // output element strides: N, spatial axes
    };
    static constexpr bool kStrided = false;
    // Per DMA instruction: the row's image offset (n, o * stride, and the lane's chunk folded
    // in) and its strided spatial position packed 16 bits per axis.
    template <int NA> struct AState { int32_t base[NA]; uint32_t pos[NA]; };

    __device__ __forceinline__ static void decompose(const Geom& geo, uint32_t m, uint32_t (&o)[NS], uint32_t& n) {
#pragma unroll
        for (int d = NS - 1; d >= 0; --d) {
            const uint32_t q = geo.odim[d].div(m);
            o[d] = m - q * geo.odim[d].d;
            m = q;
        }
        n = m;
    }

    template <typename S, int NA>
    __device__ __forceinline__ static AState<NA> a_init(const GemmArgs& g, const Geom& geo, uint32_t m0,
                                                        uint32_t rows_a, int wave, int lane) {
        constexpr int CE = 16 / sizeof(S);
        AState<NA> st;
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int r = tile::dma_row(wave, i, NA, lane);
            const uint32_t m = m0 + min((uint32_t)r, rows_a - 1);
            uint32_t o[NS], n;
            decompose(geo, m, o, n);
            int32_t base = (int32_t)(n * geo.xn) + tile::dma_chunk(r, lane) * CE;
            uint32_t pos = 0;
#pragma unroll
            for (int d = 0; d < NS; d++) {
                const uint32_t p = o[d] * (uint32_t)geo.stride[d];
                base += (int32_t)(p * geo.xs[d]);
                pos |= p << (16 * d);
            }
            st.base[i] = base;
            st.pos[i] = pos;
        }
        return st;
    }

    template <typename S, int NA>
    __device__ __forceinline__ static void a_dma(char* lds, const S* Abat, const AState<NA>& st, const GemmArgs& g,
                                                 const Geom& geo, uint32_t m0, uint32_t p, int wave, int lane) {
        constexpr int PE = tile::ROWB / sizeof(S);       // K elements per pair
        // wave-uniform: kernel position and channel block of pair p
        uint32_t kpos = geo.cpairs.div(p);
        const uint32_t cp = p - kpos * geo.cpairs.d;
        int32_t kk[NS];
        int32_t uoff = (int32_t)(cp * PE);
#pragma unroll
        for (int d = NS - 1; d >= 0; --d) {
            const uint32_t q = geo.kdim[d].div(kpos);
            const uint32_t k = kpos - q * geo.kdim[d].d;
            kpos = q;
            kk[d] = (int32_t)k * geo.dil[d] - geo.pad[d];
            uoff += kk[d] * (int32_t)geo.xs[d];
        }
#if __HIP_DEVICE_COMPILE__                               // (the buffer resource type is device-only)
        // The buffer form of the LDS DMA from the batch's image: a tap off the image takes byte
        // offset 2^31, past the resource's range, and the DMA writes zeros (the launcher keeps
        // the image below 2 GiB).  The compiler counts this form in vmcnt only (see dma_rows).
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(Abat), 0, (int)0x80000000u, 0x00020000);
#pragma unroll
        for (int i = 0; i < NA; i++) {
            bool valid = true;
#pragma unroll
            for (int d = 0; d < NS; d++) {
                const int32_t s = (int32_t)((st.pos[i] >> (16 * d)) & 0xffffu) + kk[d];
                valid = valid && (uint32_t)s < geo.idim[d];
            }
            const uint32_t off = valid ? (uint32_t)(st.base[i] + uoff) * (uint32_t)sizeof(S) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc, (__attribute__((address_space(3))) void*)(lds + (wave * NA + i) * 1024), 16, off, 0, 0, 0);
        }
#endif
    }

    __device__ __forceinline__ static uint64_t row_off(const GemmArgs& g, const Geom& geo, uint32_t row) {
        uint32_t o[NS], n;
        decompose(geo, row, o, n);
        uint64_t off = (uint64_t)n * geo.on;
#pragma unroll
        for (int d = 0; d < NS; d++) off += (uint64_t)o[d] * geo.os[d];
        return off;
    }
    template <typename S>
    __device__ __forceinline__ static bool row_vec_ok(const GemmArgs& g, const Geom& geo) {
        bool ok = ((uint64_t)geo.on * sizeof(S)) % 16 == 0;
#pragma unroll
        for (int d = 0; d < NS; d++) ok = ok && ((uint64_t)geo.os[d] * sizeof(S)) % 16 == 0;
        return ok;
    }
};

// ------------------------------------------------------------------ weight-resident halo kernel
// A "same" convolution (stride 1, each output extent equal to its input extent, 1 or 2 spatial
// axes) of a 16-bit type, one group, two or more kernel positions and at most 9 K pairs (64
// channels each, Cgp / 64 per kernel position) over all of them, whose halo saves reads (see
// halo_geom).  Output position m (flattened over batch and spatial axes) then reads, at kernel
// position t, input pixel m + sh_t (sh_t = sum_d (k_d dil_d - pad_d) x the pixel stride of axis d)
// whenever that tap lies inside the image, zeros otherwise.
//
// * The kernel stays in registers.  A workgroup of 8 waves (two per SIMD) owns a column group of
//   128 output channels; wave (wm, wn) holds the MFMA B fragments of channels 32 wn .. 32 wn + 31
//   over all of K for the workgroup's whole life (KP x 16 registers), loaded once through LDS.
// * A tile is 64 consecutive output positions.  Its A operand for all KP K pairs is one halo: the
//   input pixels m0 - rlo .. m0 + 63 + rhi, Cgp x 2 bytes each, DMA'd once into one half of a
//   two-tile LDS ring (178 rows of 128 bytes for a 3 x 3 kernel over 64 channels of 56-pixel image
//   rows, a third of the bytes of gathering every tap's 64 rows).  A fragment of tap t reads the
//   LDS rows of pixel (m - m0) + rlo + sh_t, or a zero row for a tap off the image.  The next
//   tile's halo lands while this one runs.
// * Wave (wm, wn) computes output rows 32 wm .. + 31 x its 32 channels: per K block of 16, one
//   1 KB A fragment read from LDS for one MFMA.
// * The previous tile's results, rounded to 16 bits, are stored in pieces between the current
//   tile's MFMAs: each wave stages its 32 x 32 block in its own 2 KB of LDS and stores 64-byte
//   row pieces (16 rows per instruction) instead of 16 bytes of 32 rows per instruction from the
//   fragment.  One vmcnt(0) wait per tile covers the stores and the DMA.
namespace wres {
constexpr int BM = 64;                          // output positions per tile
constexpr int BNC = 128;                        // output channels per column group
constexpr int WSLOT = BNC * tile::ROWB;         // one K pair of the group's kernel rows (16 KB)
constexpr int MAX_KP = 9;
constexpr int CAP = 512;                        // rows of one ring half (64 KB)
constexpr int RING = CAP * tile::ROWB;
constexpr int MAX_HALO = 376;                   // halo rows DMA'd per tile, at most
constexpr int ZROW = 383 * tile::ROWB;          // a row of zeros (taps off the image)
constexpr int STAGE = 384 * tile::ROWB;         // rows 384 .. 511: C staging, 2 KB per wave
// The two ring halves are separate arrays, so the compiler can tell the halo DMA into one half
// from the fragment reads of the other and adds no wait for it.  C staging uses rows of the
// current half that the DMA never writes.  Before the loop the halves stage the kernel rows: K
// pairs 0-3 in half 0, 4-7 in half 1, 8 in an array of its own.
static_assert(MAX_KP * WSLOT <= 2 * RING + WSLOT, "kernel row staging");
static_assert(2 * RING + WSLOT <= 160 * 1024, "LDS of a workgroup");
constexpr int PREFETCH = 4;                     // A fragments in flight ahead of the MFMAs

// An LDS row is one 128-byte K pair: pixel q of a halo owns rows q cp .. q cp + cp - 1 (cp = K pairs
// per pixel, Cgp / 64), and K pair p of the kernel is channel block p % cp of kernel position p / cp.
struct HaloGeom {
    FastDiv s0, s1;                 // spatial extents (1-D: s0 = 1)
    FastDiv cp;                     // K pairs per pixel
    int32_t rlo;                    // halo pixels before a tile's first position
    uint32_t hrows;                 // halo rows DMA'd per tile (a multiple of 8, <= MAX_HALO)
    uint32_t npix;                  // input pixels (batch x spatial)
    int32_t sh[MAX_KP];             // per K pair: row shift (pixel shift x cp + channel block)
    int32_t dk0[MAX_KP], dk1[MAX_KP];   // per K pair: its kernel position's offset along each axis
    uint32_t on, os0, os1;          // output element strides: batch, axis 0, axis 1
};

template <int DT> struct FragT;
template <> struct FragT<MX_FLOAT16> { using V = tile::h8v; };
template <> struct FragT<MX_BFLOAT16> { using V = tile::b8v; };

template <int DT>
__device__ __forceinline__ tile::f16v mma(const typename FragT<DT>::V& b, const typename FragT<DT>::V& a,
                                          const tile::f16v& c) {
    if constexpr (DT == MX_FLOAT16) return __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0);
}

// g.M output positions, g.N channels, g.K = KP x 64; g.tiles_m = ceil(M / 64).  Block b serves
// column group b / bpc and, within it, tiles [j T / bpc, (j + 1) T / bpc) with j = b % bpc.
// Eight waves, two per SIMD: wave (wm, wn) computes output rows 32 wm .. + 31 x channels
// 32 wn .. + 31 of the group and holds those channels' kernel fragments (KP x 16 registers).  One
// wave per SIMD holding 64 channels (two MFMAs per A fragment read) kept the matrix cores busy
// only about half the time: a lone wave's MFMAs issue one after another with gaps that a second
// wave fills.
// CP1: one K pair per pixel (cp = 1, 64 channels), with the pair arithmetic folded away.
template <int DT, int KP, bool CP1>
__global__ __launch_bounds__(512) void conv_halo_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ xp,
                                                        const uint16_t* __restrict__ wp, GemmArgs ga, HaloGeom hga,
                                                        uint32_t bpc) {
    using S = uint16_t;
    using V = typename FragT<DT>::V;
    constexpr int NW = 8;                       // waves
    constexpr int KB = 4 * KP;                  // K blocks of 16 elements
    constexpr int PE = tile::ROWB / 2;          // elements per K pair
    __shared__ __align__(16) char ring0[RING];
    __shared__ __align__(16) char ring1[RING];
    __shared__ __align__(16) char wtail[KP > 8 ? WSLOT : 16];
    auto wslot = [&](int p) -> char* { return p < 4 ? ring0 + p * WSLOT : p < 8 ? ring1 + (p - 4) * WSLOT : wtail; };
    // the arguments as plain values: lambdas that capture a by-value kernel argument struct make
    // the compiler copy it to scratch memory
    struct {
        uint32_t M, N, K, tiles_m;
    } g = {ga.M, ga.N, ga.K, ga.tiles_m};
    struct {
        FastDiv s0, s1, cp;
        int32_t rlo;
        uint32_t hrows, npix, on, os0, os1;
        int32_t sh[KP], dk0[KP], dk1[KP];
    } hg;
    hg.s0 = hga.s0;
    hg.s1 = hga.s1;
    hg.cp = hga.cp;
    hg.rlo = hga.rlo;
    hg.hrows = hga.hrows;
    hg.npix = hga.npix;
    hg.on = hga.on;
    hg.os0 = hga.os0;
    hg.os1 = hga.os1;
#pragma unroll
    for (int p = 0; p < KP; p++) {
        hg.sh[p] = hga.sh[p];
        hg.dk0[p] = hga.dk0[p];
        hg.dk1[p] = hga.dk1[p];
    }

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 2, wn = wave & 3, r32 = lane & 31, h = lane >> 5;
    const uint32_t cg = blockIdx.x / bpc, j = blockIdx.x - cg * bpc;
    const uint32_t n0 = cg * BNC;
    const uint32_t t_lo = (uint32_t)((uint64_t)j * g.tiles_m / bpc);
    const uint32_t t_hi = (uint32_t)((uint64_t)(j + 1) * g.tiles_m / bpc);

    // kernel rows of the column group -> LDS (pair p in wslot(p), 128 rows of 128 bytes) -> registers
    const uint32_t rows_b = g.N - n0 < (uint32_t)BNC ? g.N - n0 : (uint32_t)BNC;
    {
        const S* wcg = wp + (uint64_t)n0 * g.K;
        const auto ob = tile::dma_offsets<S, 2>(rows_b, g.K, wave, lane);
#pragma unroll
        for (int p = 0; p < KP; p++) tile::dma_rows<S, 2>(wslot(p), wcg, ob, (uint32_t)(p * PE), wave);
    }
    tile::wait_vmem<0>();
    __syncthreads();
    V bf[KB];
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
        const int rb = 32 * wn + r32;
        bf[kb] = *reinterpret_cast<const V*>(wslot(kb / 4) + rb * tile::ROWB + tile::swz(rb, 2 * (kb % 4) + h) * 16);
    }
    __syncthreads();                            // every wave holds its fragments: the ring is free
    if (wave == 0 && lane < 16) *reinterpret_cast<uint4*>((lane < 8 ? ring0 : ring1) + ZROW + (lane % 8) * 16) = uint4{0, 0, 0, 0};

#if __HIP_DEVICE_COMPILE__                               // (the buffer resource type is device-only)
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<S*>(xp), 0, (int)(hg.npix * (CP1 ? 1u : hg.cp.d) * (uint32_t)tile::ROWB), 0x00020000);
#endif
    // the halo of tile t: row r = 0 .. hrows - 1 is channel block r % cp of input pixel
    // m0 - rlo + r / cp (clamped into the image: a clamped pixel is read only by taps off the image,
    // which take the zero row); DMA instruction i fills rows 8 i .. 8 i + 7, lane L row 8 i + L / 8,
    // stored chunk L % 8
    auto issue_a = [&](uint32_t t, char* buf) __attribute__((always_inline)) {
        const int32_t first = (int32_t)(t * BM) - hg.rlo;
        const int nd = (int)(hg.hrows / 8);
        for (int i = wave; i < nd; i += NW) {
            const uint32_t r = (uint32_t)(8 * i + lane / 8);
            const uint32_t rq = CP1 ? r : hg.cp.div(r), blk = CP1 ? 0u : r - rq * hg.cp.d;
            int32_t pix = first + (int32_t)rq;
            pix = pix < 0 ? 0 : (pix >= (int32_t)hg.npix ? (int32_t)hg.npix - 1 : pix);
            const uint32_t off = ((uint32_t)pix * (CP1 ? 1u : hg.cp.d) + blk) * (uint32_t)tile::ROWB +
                                 (uint32_t)tile::swz((int)r, lane % 8) * 16u;
#if __HIP_DEVICE_COMPILE__
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(buf + i * 1024),
                                                     16, off, 0, 0, 0);
#else
            (void)off;
#endif
        }
    };
    // acc: the tile as a C^T fragment (lane: row r32 of the wave's 32, columns 8 q + 4 h + e in
    // register 4 q + e); prev: the finished previous tile rounded to 16 bits, two columns a word
    // (word 2 q + i: columns 8 q + 4 h + 2 i, + 1), stored during the next tile's MFMAs
    tile::f16v acc;
    uint32_t prev[8];
    const uint32_t cw = n0 + 32 * wn;
    const bool full_cols = cw + 32 <= g.N;
    auto row_off = [&](uint32_t m) __attribute__((always_inline)) -> uint64_t {
        const uint32_t q1 = hg.s1.div(m), o1 = m - q1 * hg.s1.d;
        const uint32_t n = hg.s0.div(q1), o0 = q1 - n * hg.s0.d;
        return (uint64_t)n * hg.on + (uint64_t)o0 * hg.os0 + (uint64_t)o1 * hg.os1;
    };
    auto cvt = [](float v) __attribute__((always_inline)) -> uint16_t {
        return DT == MX_FLOAT16 ? float_to_half_bits(v) : float_to_bf16(v);
    };
    // staged store of a finished tile (the wave's 32 rows x 32 channels, 64 bytes a row), in 7
    // pieces: 4 that write its fragment to the wave's 2 KB of LDS (piece q: registers 4 q ..;
    // chunk k of row r at (k ^ (r & 3)) * 16), a compiler fence, then 2 that each read 16 rows back
    // and store them (64 lanes x 16 bytes).  A wave's LDS accesses complete in order, so the reads
    // see the writes; stage and rows are this wave's own, and the barrier at the top of the next
    // tile orders them against the DMA.
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    auto store_piece = [&](char* stage, const uint32_t (&c)[8], uint32_t mw, int j) __attribute__((always_inline)) {
        if (j < 4) {
            const int q = j;
            uint2 u;
            u.x = c[2 * q];
            u.y = c[2 * q + 1];
            // (as inline asm: the compiler waited for the pending halo DMA before this write, which
            // goes to rows that DMA never touches)
            const uint32_t addr = (uint32_t)(uintptr_t)(stage + r32 * 64 + ((q ^ (r32 & 3)) * 16) + 8 * h);
            asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(u) : "memory");
        } else if (j == 4) {
            asm volatile("" ::: "memory");
        } else {
            const int it = j - 5, k = lane % 4, rr = 16 * it + lane / 4;
            const u4v v = *reinterpret_cast<const u4v*>(stage + rr * 64 + ((k ^ (rr & 3)) * 16));
            if (mw + rr < g.M)
                __builtin_nontemporal_store(v, reinterpret_cast<u4v*>(out + row_off(mw + rr) + cw + 8 * k));
        }
    };
    constexpr int PIECES = 7;
    // a column group's last waves may hold fewer than 32 channels: element stores from the fragment
    auto store_edge = [&](const uint32_t (&c)[8], uint32_t t) __attribute__((always_inline)) {
        const uint32_t row = t * BM + 32 * wm + r32;
        if (row >= g.M) return;
        S* crow = out + row_off(row);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t col = cw + 8 * q + 4 * h + e;
                if (col < g.N) crow[col] = (uint16_t)(c[2 * q + e / 2] >> (16 * (e % 2)));
            }
    };
    auto store_all = [&](auto full, const uint32_t (&c)[8], uint32_t t) __attribute__((always_inline)) {
        if constexpr (decltype(full)::value) {
#pragma unroll
            for (int j = 0; j < PIECES; j++) store_piece(ring0 + STAGE + wave * 2048, c, t * BM + 32 * wm, j);
        } else {
            store_edge(c, t);
        }
    };
    // Tile t from ring half P; with HP, tile t - 1's results (prev) are stored meanwhile -- with
    // FULL in pieces between its MFMAs, otherwise before them.
    auto step = [&](auto par, auto has_prev, auto full, uint32_t t) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;
        constexpr bool HP = decltype(has_prev)::value, FULL = decltype(full)::value;
        char* cur = P == 0 ? ring0 : ring1;
        char* nxt = P == 0 ? ring1 : ring0;
        char* stage = cur + STAGE + wave * 2048;
        tile::wait_vmem<0>();                   // this wave's DMA of tile t (and its last stores)
        tile::ring_barrier();                   // every wave's DMA of t landed; t - 1's reads done
        if (t + 1 < t_hi) issue_a(t + 1, nxt);
        if constexpr (HP && !FULL) store_edge(prev, t - 1);
        // per tap: the LDS byte offset of this lane's A row (its output position's tap pixel, or
        // the zero row) and that row's chunk swizzle
        const uint32_t m = t * BM + 32 * wm + r32;
        const uint32_t q1 = hg.s1.div(m), o1 = m - q1 * hg.s1.d;
        const uint32_t o0 = q1 - hg.s0.div(q1) * hg.s0.d;
        const int base = (32 * wm + r32 + hg.rlo) * (CP1 ? 1 : (int)hg.cp.d);
        int roff[KP], rsw[KP];
#pragma unroll
        for (int p = 0; p < KP; p++) {
            const bool ok = (uint32_t)((int32_t)o0 + hg.dk0[p]) < hg.s0.d && (uint32_t)((int32_t)o1 + hg.dk1[p]) < hg.s1.d;
            const int row = base + hg.sh[p];
            roff[p] = ok ? row * tile::ROWB : ZROW;
            rsw[p] = ok ? (row >> 1) & 7 : 0;
        }
        auto rd = [&](int kb) __attribute__((always_inline)) -> V {
            const int p = kb / 4;
            return *reinterpret_cast<const V*>(cur + roff[p] + (((2 * (kb % 4) + h) ^ rsw[p]) * 16));
        };
        const uint32_t mw = (t - 1) * BM + 32 * wm;     // tile t - 1's first row of this wave (HP)
        V a[PREFETCH];
#pragma unroll
        for (int i = 0; i < PREFETCH; i++) a[i] = rd(i);
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.0f;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            acc = mma<DT>(bf[kb], a[kb % PREFETCH], acc);
            if (kb + PREFETCH < KB) a[kb % PREFETCH] = rd(kb + PREFETCH);
            if constexpr (HP && FULL) {
                // piece j goes after the MFMA of K block min(2 j + 2, KB - 1)
#pragma unroll
                for (int j = 0; j < PIECES; j++)
                    if ((2 * j + 2 < KB ? 2 * j + 2 : KB - 1) == kb) store_piece(stage, prev, mw, j);
            }
        }
#pragma unroll
        for (int w = 0; w < 8; w++) prev[w] = (uint32_t)cvt(acc[2 * w]) | ((uint32_t)cvt(acc[2 * w + 1]) << 16);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using BF = std::false_type;
    using BT = std::true_type;
    auto run = [&](auto full) __attribute__((always_inline)) {
        uint32_t t = t_lo;
        step(I0{}, BF{}, full, t);
        for (;;) {
            if (++t >= t_hi) {
                store_all(full, prev, t - 1);
                break;
            }
            step(I1{}, BT{}, full, t);
            if (++t >= t_hi) {
                store_all(full, prev, t - 1);
                break;
            }
            step(I0{}, BT{}, full, t);
        }
    };
    if (t_lo >= t_hi) return;                   // (uniform over the block)
    issue_a(t_lo, ring0);
    if (full_cols) run(BT{});
    else run(BF{});
}
}  // namespace wres

// ------------------------------------------------------------------ packing
struct ConvShape {
    int ns;
    uint32_t N, C, O, groups, Cg, Og;
    uint32_t S[kMaxSpatial], K[kMaxSpatial], OS[kMaxSpatial];
    uint64_t in_s[kMaxSpatial + 2], k_s[kMaxSpatial + 2], out_s[kMaxSpatial + 2];
};

// Xp[n, s.., g, c] = c < Cg ? in[n, s.., g Cg + c] : 0, one element per thread.
struct PackInDesc {
    int ns;
    FastDiv dims[kMaxSpatial + 2];       // N, S.., groups * Cgp  (outermost first)
    FastDiv cgp;
    uint32_t Cg;
    uint64_t s[kMaxSpatial + 2];         // input strides: N, spatial axes, channel
};

template <typename S>
__global__ __launch_bounds__(256) void pack_input_kernel(S* __restrict__ xp, const S* __restrict__ in, uint64_t total,
                                                         PackInDesc d) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += stride) {
        uint64_t rem = t;
        const uint64_t gc = rem % d.dims[d.ns + 1].d;
        rem /= d.dims[d.ns + 1].d;
        uint64_t off = 0;
        for (int a = d.ns; a >= 1; --a) {
            off += (rem % d.dims[a].d) * d.s[a];
            rem /= d.dims[a].d;
        }
        off += rem * d.s[0];
        const uint32_t g = d.cgp.div((uint32_t)gc);
        const uint32_t c = (uint32_t)gc - g * d.cgp.d;
        xp[t] = c < d.Cg ? in[off + (uint64_t)(g * d.Cg + c) * d.s[d.ns + 1]] : S(0);
    }
}

// Channel-major image (the spatial axes form one unit-stride run P, channels at stride sC, as an
// NCHW tensor viewed NHWC): Xp[n, p, c] = in[n, c, p] as a tiled transpose through LDS, 64 x 64
// per block, reads and writes both along their contiguous axis.  groups == 1 here.
template <typename S>
__global__ __launch_bounds__(256) void pack_input_transpose_kernel(S* __restrict__ xp, const S* __restrict__ in,
                                                                   uint32_t P, uint32_t C, uint32_t Cgp, uint64_t sN,
                                                                   uint64_t sC) {
    __shared__ S t[64][65];
    const uint32_t p0 = blockIdx.x * 64, c0 = blockIdx.y * 64, n = blockIdx.z;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const S* src = in + (uint64_t)n * sN;
#pragma unroll
    for (int i = 0; i < 16; i++) {                  // read: 64 channels x 64 positions
        const uint32_t c = c0 + ty + 4 * i, p = p0 + tx;
        t[ty + 4 * i][tx] = (c < C && p < P) ? src[(uint64_t)c * sC + p] : S(0);
    }
    __syncthreads();
    S* dst = xp + (uint64_t)n * P * Cgp;
#pragma unroll
    for (int i = 0; i < 16; i++) {                  // write: 64 positions x 64 channels
        const uint32_t p = p0 + ty + 4 * i, c = c0 + tx;
        if (p < P && c < Cgp) dst[(uint64_t)p * Cgp + c] = t[tx][ty + 4 * i];
    }
}

// The same transpose with 16-byte accesses on both sides (positions per image, channel stride,
// image stride and the source all in whole 16-byte units).  Lane (cb = l % 8, pb = l / 8) of wave
// w loads VE channel rows (VE = elements per 16 bytes) of VE consecutive positions, transposes the
// VE x VE block in registers and stores VE position rows of VE channels: per instruction, 8 lanes
// cover 128 contiguous bytes of one channel row (loads) or of one position row (stores).
// Channels in [C, Cgp) are written as zeros.
template <typename S>
__device__ __forceinline__ void pack_input_transpose16_body(S* __restrict__ xp, const S* __restrict__ in, uint32_t P,
                                                            uint32_t C, uint32_t Cgp, uint64_t sN, uint64_t sC,
                                                            uint32_t bx, uint32_t by, uint32_t bz) {
    constexpr int VE = 16 / sizeof(S);
    struct alignas(16) V { S v[VE]; };
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t c = by * (8 * VE) + (lane & 7) * VE;
    const uint32_t p = (bx * 32 + wave * 8 + (lane >> 3)) * VE;
    if (p >= P || c >= Cgp) return;
    const S* src = in + (uint64_t)bz * sN + p;
    // rows past C load a valid row (no branch between the loads) and are zeroed afterwards
    V v[VE];
#pragma unroll
    for (int i = 0; i < VE; i++) v[i] = *reinterpret_cast<const V*>(src + (uint64_t)min(c + i, C - 1) * sC);
#pragma unroll
    for (int i = 0; i < VE; i++)
        if (c + i >= C) {
#pragma unroll
            for (int j = 0; j < VE; j++) v[i].v[j] = S(0);
        }
    S* dst = xp + ((uint64_t)bz * P + p) * Cgp + c;
#pragma unroll
    for (int j = 0; j < VE; j++) {
        V w;
#pragma unroll
        for (int i = 0; i < VE; i++) w.v[i] = v[i].v[j];
        *reinterpret_cast<V*>(dst + (uint64_t)j * Cgp) = w;
    }
}

template <typename S>
__global__ __launch_bounds__(256) void pack_input_transpose16_kernel(S* __restrict__ xp, const S* __restrict__ in,
                                                                     uint32_t P, uint32_t C, uint32_t Cgp, uint64_t sN,
                                                                     uint64_t sC) {
    pack_input_transpose16_body(xp, in, P, C, Cgp, sN, sC, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Wp[o, k.., c] = c < Cg ? kern[o, (flip ? K - 1 - k : k).., c] : 0.
struct PackKDesc {
    int ns;
    FastDiv dims[kMaxSpatial + 2];       // O, K.., Cgp
    uint32_t K[kMaxSpatial];
    uint32_t Cg;
    int flip;
    uint64_t s[kMaxSpatial + 2];
};

// The launcher keeps total below 2^32, so the index decomposes with 32-bit FastDiv.
template <typename S>
__device__ __forceinline__ void pack_kernel_body(S* __restrict__ wp, const S* __restrict__ kern, uint32_t total,
                                                 const PackKDesc& d, uint32_t first, uint32_t stride) {
    for (uint32_t t = first; t < total; t += stride) {
        uint32_t rem = t;
        uint32_t q = d.dims[d.ns + 1].div(rem);
        const uint32_t c = rem - q * d.dims[d.ns + 1].d;
        rem = q;
        uint64_t off = (uint64_t)c * d.s[d.ns + 1];
        for (int a = d.ns; a >= 1; --a) {
            q = d.dims[a].div(rem);
            const uint32_t k = rem - q * d.dims[a].d;
            rem = q;
            off += (uint64_t)(d.flip ? d.K[a - 1] - 1 - k : k) * d.s[a];
        }
        off += (uint64_t)rem * d.s[0];
        wp[t] = c < d.Cg ? kern[off] : S(0);
    }
}

template <typename S>
__global__ __launch_bounds__(256) void pack_kernel_kernel(S* __restrict__ wp, const S* __restrict__ kern,
                                                          uint32_t total, PackKDesc d) {
    pack_kernel_body(wp, kern, total, d, blockIdx.x * 256 + threadIdx.x, gridDim.x * 256);
}

// Both packs in one launch (a channel-major input and a kernel to pack, the reference's NCHW /
// OIHW views), as a 1-D grid: the first nwb blocks pack the kernel, one element per thread; the
// rest are the (gx, gy, N) blocks of pack_input_transpose16_kernel, x fastest.
template <typename S>
__global__ __launch_bounds__(256) void pack_input16_and_kernel_kernel(S* __restrict__ xp, const S* __restrict__ in,
                                                                      uint32_t P, uint32_t C, uint32_t Cgp, uint64_t sN,
                                                                      uint64_t sC, uint32_t gx, uint32_t gy,
                                                                      S* __restrict__ wp, const S* __restrict__ kern,
                                                                      uint32_t wtotal, uint32_t nwb, PackKDesc d) {
    const uint32_t b = blockIdx.x;
    if (b < nwb) {
        pack_kernel_body(wp, kern, wtotal, d, b * 256 + threadIdx.x, nwb * 256);
        return;
    }
    const uint32_t r = b - nwb;
    const uint32_t q = r / gx;
    pack_input_transpose16_body(xp, in, P, C, Cgp, sN, sC, r - q * gx, q % gy, q / gy);
}

// A 1 x 1 kernel with stride > 1 and no padding reads only the sampled positions: pack just
// those, Xp[n, o.., c] = c < C ? in[n, (o * stride).., c] : 0, so the product runs at stride 1 on
// a dense [N, OS.., Cgp] input.  Lane (cb = l % 8, pb = l / 8) of wave w takes output position
// 32 x + 8 w + pb and the VE channels starting at (8 y + cb) VE: the 8 lanes of one position
// store 128 contiguous bytes of its row, and the 8 positions of one channel read neighbouring
// samples.  osd: FastDiv of the last output extent (2-D); ns = 1 or 2.
template <typename S>
__global__ __launch_bounds__(256) void pack_input_sampled_kernel(S* __restrict__ xp, const S* __restrict__ in,
                                                                 uint32_t OP, FastDiv osd, int ns, uint32_t C,
                                                                 uint32_t Cgp, uint64_t sN, uint64_t sC, uint64_t s1,
                                                                 uint64_t s2, uint32_t st1, uint32_t st2) {
    constexpr int VE = 16 / sizeof(S);
    struct alignas(16) V { S v[VE]; };
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = blockIdx.x * 32 + wave * 8 + (lane >> 3);
    const uint32_t c0 = (blockIdx.y * 8 + (lane & 7)) * VE;
    if (q >= OP || c0 >= Cgp) return;
    uint64_t off;
    if (ns == 2) {
        const uint32_t oh = osd.div(q), ow = q - oh * osd.d;
        off = (uint64_t)oh * st1 * s1 + (uint64_t)ow * st2 * s2;
    } else {
        off = (uint64_t)q * st1 * s1;
    }
    const S* src = in + (uint64_t)blockIdx.z * sN + off;
    // channels past C load channel C - 1 (no branch between the loads) and are zeroed after
    V v;
#pragma unroll
    for (int i = 0; i < VE; i++) v.v[i] = src[(uint64_t)min(c0 + i, C - 1) * sC];
#pragma unroll
    for (int i = 0; i < VE; i++)
        if (c0 + i >= C) v.v[i] = S(0);
    *reinterpret_cast<V*>(xp + ((uint64_t)blockIdx.z * OP + q) * Cgp + c0) = v;
}

// The same sampled pack for a channel-major image (the reference's NCHW tensors seen channels-last:
// positions contiguous along the last spatial axis, channels far apart), where reading a channel
// run per lane touches one line per element.  A block takes 64 output positions x 64 channels of
// one image: lane q of every wave loads sampled position q of its channels -- consecutive lanes,
// neighbouring samples of one channel row -- into an LDS tile [position][channel dword] (rows of
// DPR + 1 dwords, so the 64 lanes' writes land in distinct banks); then each thread stores whole
// 16-byte runs of 4 dwords of a position row.  Channels in [C, Cgp) are written as zeros.
template <typename S>
__global__ __launch_bounds__(256) void pack_input_sampled_cm_kernel(S* __restrict__ xp, const S* __restrict__ in,
                                                                    uint32_t OP, FastDiv osd, int ns, uint32_t C,
                                                                    uint32_t Cgp, uint64_t sN, uint64_t sC, uint64_t s1,
                                                                    uint64_t s2, uint32_t st1, uint32_t st2) {
    constexpr int EPD = 4 / (int)sizeof(S);          // channels per dword
    constexpr int DPR = 64 / EPD;                     // dwords of a 64-channel position row
    constexpr int LD = DPR + 1;                       // padded LDS row (dwords)
    __shared__ uint32_t tile[64 * LD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    // phase 1: lane = position, dword columns wave, wave + 4, ...
    {
        const uint32_t q = min(q0 + (uint32_t)lane, OP - 1);
        uint64_t off;
        if (ns == 2) {
            const uint32_t oh = osd.div(q), ow = q - oh * osd.d;
            off = (uint64_t)oh * st1 * s1 + (uint64_t)ow * st2 * s2;
        } else {
            off = (uint64_t)q * st1 * s1;
        }
        const S* src = in + (uint64_t)blockIdx.z * sN + off;
#pragma unroll
        for (int i = 0; i < DPR / 4; i++) {
            const int d = wave + 4 * i;
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < EPD; e++) {
                const uint32_t c = c0 + (uint32_t)(d * EPD + e);
                S v = src[(uint64_t)min(c, C - 1) * sC];
                if (c >= C) v = S(0);
                uint32_t bitsv = 0;
                __builtin_memcpy(&bitsv, &v, sizeof(S));
                word |= bitsv << (8 * sizeof(S) * e);
            }
            tile[lane * LD + d] = word;
        }
    }
    __syncthreads();
    // phase 2: 16-byte chunk k (dwords 4 k .. 4 k + 3) of position row r
    constexpr int CPR = DPR / 4;                      // chunks per position row
#pragma unroll
    for (int i = 0; i < 64 * CPR / 256; i++) {
        const int idx = (int)threadIdx.x + 256 * i;
        const int r = idx / CPR, k = idx % CPR;
        const uint32_t q = q0 + (uint32_t)r, c = c0 + (uint32_t)(4 * k * EPD);
        if (q >= OP || c >= Cgp) continue;
        uint4 v;
        v.x = tile[r * LD + 4 * k];
        v.y = tile[r * LD + 4 * k + 1];
        v.z = tile[r * LD + 4 * k + 2];
        v.w = tile[r * LD + 4 * k + 3];
        *reinterpret_cast<uint4*>(xp + ((uint64_t)blockIdx.z * OP + q) * Cgp + c) = v;
    }
}

// ------------------------------------------------------------------ direct kernel
struct DirectDesc {
    int ns;
    uint32_t N, O, Cg, Og, groups;
    uint32_t S[kMaxSpatial], K[kMaxSpatial], OS[kMaxSpatial];
    int32_t pad[kMaxSpatial], stride[kMaxSpatial], dil[kMaxSpatial], dil_lhs[kMaxSpatial];
    uint64_t in_s[kMaxSpatial + 2], k_s[kMaxSpatial + 2], out_s[kMaxSpatial + 2];
    int flip;
    uint64_t kdot;                       // prod K * Cg
};

template <int DT>
__global__ __launch_bounds__(256) void conv_direct_kernel(typename dt_traits<DT>::S* __restrict__ out,
                                                          const typename dt_traits<DT>::S* __restrict__ in,
                                                          const typename dt_traits<DT>::S* __restrict__ kern,
                                                          uint64_t total, DirectDesc d) {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    const uint64_t gstride = (uint64_t)gridDim.x * 256;
    for (uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += gstride) {
        // t -> (n, o_1 .. o_ns, oc), oc fastest
        uint64_t rem = t;
        const uint32_t oc = (uint32_t)(rem % d.O);
        rem /= d.O;
        int64_t base[kMaxSpatial];
        uint64_t out_off = (uint64_t)oc * d.out_s[d.ns + 1];
        for (int a = d.ns - 1; a >= 0; --a) {
            const uint32_t o = (uint32_t)(rem % d.OS[a]);
            rem /= d.OS[a];
            base[a] = (int64_t)o * d.stride[a] - d.pad[a];
            out_off += (uint64_t)o * d.out_s[a + 1];
        }
        const uint64_t n = rem;
        out_off += n * d.out_s[0];
        const uint32_t c0 = (oc / d.Og) * d.Cg;
        using Acc = std::conditional_t<Tr::is_float, float, uint64_t>;
        Acc acc = 0;
        for (uint64_t tt = 0; tt < d.kdot; tt++) {
            const uint32_t c = (uint32_t)(tt % d.Cg);
            uint64_t rk = tt / d.Cg;
            uint64_t ioff = n * d.in_s[0] + (uint64_t)(c0 + c) * d.in_s[d.ns + 1];
            uint64_t koff = (uint64_t)oc * d.k_s[0] + (uint64_t)c * d.k_s[d.ns + 1];
            bool valid = true;
            for (int j = d.ns - 1; j >= 0; --j) {
                const int64_t kj = (int64_t)(rk % d.K[j]);
                rk /= d.K[j];
                const int64_t s = base[j] + kj * d.dil[j];
                const int64_t len = ((int64_t)d.S[j] - 1) * d.dil_lhs[j] + 1;
                if (s < 0 || s >= len || (s % d.dil_lhs[j]) != 0) { valid = false; break; }
                const int64_t kr = d.flip ? ((int64_t)d.K[j] - 1 - kj) : kj;
                koff += (uint64_t)kr * d.k_s[j + 1];
                ioff += (uint64_t)(s / d.dil_lhs[j]) * d.in_s[j + 1];
            }
            if (!valid) continue;
            if constexpr (Tr::is_float) {
                acc = __builtin_fmaf(Tr::ld(kern[koff]), Tr::ld(in[ioff]), acc);
            } else {
                acc += (uint64_t)(int64_t)kern[koff] * (uint64_t)(int64_t)in[ioff];
            }
        }
        if constexpr (Tr::is_float) out[out_off] = Tr::st(acc);
        else out[out_off] = (S)acc;
    }
}

// ------------------------------------------------------------------ planning
struct Plan {
    bool mfma = false;
    bool pack_in = false, pack_k = false;
    uint32_t Cgp = 0;
    size_t xp_bytes = 0, wp_bytes = 0;
};

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

bool contiguous_channels_last(int ns, const uint32_t* shape, const uint64_t* s) {
    uint64_t want = 1;
    for (int a = ns + 1; a >= 0; --a) {
        if (shape[a] != 1 && s[a] != want) return false;
        want *= shape[a];
    }
    return true;
}

// The MFMA plan as far as the shapes and strides decide it (flip, dilations and pointer
// alignment are checked again at launch).
Plan plan_conv(int dtype, const ConvShape& cs) {
    Plan p;
    if (!(dtype == MX_FLOAT32 || dtype == MX_FLOAT16 || dtype == MX_BFLOAT16)) return p;
    if (cs.ns < 1 || cs.ns > 2) return p;
    const size_t es = dtype_size(dtype);
    const uint32_t PE = (uint32_t)(tile::ROWB / es);
    p.Cgp = (cs.Cg + PE - 1) / PE * PE;
    uint64_t sp = 1, kp = 1, osp = 1;
    for (int d = 0; d < cs.ns; d++) {
        sp *= cs.S[d];
        kp *= cs.K[d];
        osp *= cs.OS[d];
        if (cs.S[d] >= 32768 || (uint64_t)cs.OS[d] * 1 >= 32768) return p;
    }
    const uint64_t xp_elems = (uint64_t)cs.N * sp * cs.groups * p.Cgp;
    const uint64_t K = kp * p.Cgp;
    const uint64_t M = (uint64_t)cs.N * osp;
    if (xp_elems * es >= (1ull << 31) || K >= (1ull << 31) || M >= (1ull << 32) || K * es * 256 >= (1ull << 32))
        return p;
    uint32_t ishape[kMaxSpatial + 2], kshape[kMaxSpatial + 2];
    ishape[0] = cs.N;
    kshape[0] = cs.O;
    for (int d = 0; d < cs.ns; d++) { ishape[d + 1] = cs.S[d]; kshape[d + 1] = cs.K[d]; }
    ishape[cs.ns + 1] = cs.C;
    kshape[cs.ns + 1] = cs.Cg;
    p.pack_in = !(p.Cgp == cs.Cg && contiguous_channels_last(cs.ns, ishape, cs.in_s));
    p.pack_k = !(p.Cgp == cs.Cg && contiguous_channels_last(cs.ns, kshape, cs.k_s));
    p.xp_bytes = p.pack_in ? align256(xp_elems * es) : 0;
    p.wp_bytes = align256((uint64_t)cs.O * K * es);      // flip is unknown here: always counted
    p.mfma = true;
    return p;
}

int read_shape(int dtype, int ns, const uint32_t* in_shape, const uint32_t* k_shape, const uint32_t* out_shape,
               const uint32_t* in_strides, const uint32_t* k_strides, const uint32_t* out_strides, int groups,
               ConvShape& cs, const char* who) {
    if (ns < 1 || ns > kMaxSpatial)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": nspatial " + std::to_string(ns) + " outside [1, 6]");
    if (!in_shape || !k_shape || !out_shape || !in_strides || !k_strides || !out_strides)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null descriptor");
    if (groups < 1) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": groups must be >= 1");
    cs.ns = ns;
    cs.N = in_shape[0];
    cs.C = in_shape[ns + 1];
    cs.O = k_shape[0];
    cs.Cg = k_shape[ns + 1];
    cs.groups = (uint32_t)groups;
    if (out_shape[0] != cs.N || out_shape[ns + 1] != cs.O)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": output batch / channels do not match input / kernel");
    if ((uint64_t)cs.Cg * cs.groups != cs.C || cs.O % cs.groups != 0)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": channels do not divide into groups");
    cs.Og = cs.O / cs.groups;
    for (int d = 0; d < ns; d++) {
        cs.S[d] = in_shape[d + 1];
        cs.K[d] = k_shape[d + 1];
        cs.OS[d] = out_shape[d + 1];
    }
    for (int a = 0; a < ns + 2; a++) {
        cs.in_s[a] = in_strides[a];
        cs.k_s[a] = k_strides[a];
        cs.out_s[a] = out_strides[a];
    }
    (void)dtype;
    return MX_OK;
}

// Channel-major input (the spatial axes collapse into one unit-stride run).
bool channel_major(const ConvShape& cs, uint64_t* P) {
    bool run = cs.groups == 1 && cs.in_s[cs.ns] == 1;
    for (int d = cs.ns - 1; d >= 1 && run; --d) run = cs.in_s[d] == cs.in_s[d + 1] * cs.S[d];
    *P = 1;
    for (int d = 0; d < cs.ns; d++) *P *= cs.S[d];
    return run && *P < (1ull << 31) && cs.N < 65536;
}

// The 16-byte transpose applies (positions, strides and buffers in whole 16-byte units): its grid.
template <typename S>
bool transpose16_grid(const ConvShape& cs, uint32_t Cgp, const S* xp, const S* in, dim3* grid, uint64_t* P) {
    constexpr uint32_t VE = 16 / sizeof(S);
    if (!channel_major(cs, P) || *P % VE || cs.in_s[cs.ns + 1] % VE || cs.in_s[0] % VE || Cgp % VE ||
        (uintptr_t)in % 16 || (uintptr_t)xp % 16)
        return false;
    *grid = dim3((uint32_t)((*P + 32 * VE - 1) / (32 * VE)), (Cgp + 8 * VE - 1) / (8 * VE), cs.N);
    return true;
}

template <typename S>
int launch_pack_input(const ConvShape& cs, uint32_t Cgp, S* xp, const S* in, hipStream_t st) {
    uint64_t P;
    dim3 grid;
    if (transpose16_grid(cs, Cgp, xp, in, &grid, &P)) {
        hipLaunchKernelGGL((pack_input_transpose16_kernel<S>), grid, dim3(256), 0, st, xp, in, (uint32_t)P, cs.C, Cgp,
                           cs.in_s[0], cs.in_s[cs.ns + 1]);
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    const bool run = channel_major(cs, &P);
    if (run) {
        grid = dim3((uint32_t)((P + 63) / 64), (Cgp + 63) / 64, cs.N);
        hipLaunchKernelGGL((pack_input_transpose_kernel<S>), grid, dim3(256), 0, st, xp, in, (uint32_t)P, cs.C, Cgp,
                           cs.in_s[0], cs.in_s[cs.ns + 1]);
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    PackInDesc d{};
    d.ns = cs.ns;
    d.dims[0] = FastDiv(cs.N);
    for (int a = 0; a < cs.ns; a++) d.dims[a + 1] = FastDiv(cs.S[a]);
    d.dims[cs.ns + 1] = FastDiv(cs.groups * Cgp);
    d.cgp = FastDiv(Cgp);
    d.Cg = cs.Cg;
    for (int a = 0; a < cs.ns + 2; a++) d.s[a] = cs.in_s[a];
    const uint64_t total = (uint64_t)cs.N * P * cs.groups * Cgp;
    const uint64_t want = (total + 255) / 256;
    hipLaunchKernelGGL((pack_input_kernel<S>), dim3((uint32_t)(want < 65536 ? want : 65536)), dim3(256), 0, st, xp,
                       in, total, d);
    MX_HIP(hipGetLastError());
    return MX_OK;
}

int pack_kernel_desc(const ConvShape& cs, uint32_t Cgp, int flip, PackKDesc& d, uint64_t& total) {
    d = PackKDesc{};
    d.ns = cs.ns;
    d.dims[0] = FastDiv(cs.O);
    total = (uint64_t)cs.O * Cgp;
    for (int a = 0; a < cs.ns; a++) {
        d.dims[a + 1] = FastDiv(cs.K[a]);
        d.K[a] = cs.K[a];
        total *= cs.K[a];
    }
    d.dims[cs.ns + 1] = FastDiv(Cgp);
    d.Cg = cs.Cg;
    d.flip = flip;
    for (int a = 0; a < cs.ns + 2; a++) d.s[a] = cs.k_s[a];
    if (total > 0xffffffffull) return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: kernel of 2^32 or more elements");
    return MX_OK;
}

template <typename S>
int launch_pack_kernel(const ConvShape& cs, uint32_t Cgp, int flip, S* wp, const S* kern, hipStream_t st) {
    PackKDesc d;
    uint64_t total;
    if (int rc = pack_kernel_desc(cs, Cgp, flip, d, total)) return rc;
    const uint64_t want = (total + 255) / 256;
    hipLaunchKernelGGL((pack_kernel_kernel<S>), dim3((uint32_t)(want < 65536 ? want : 65536)), dim3(256), 0, st, wp,
                       kern, (uint32_t)total, d);
    MX_HIP(hipGetLastError());
    return MX_OK;
}

// The weight-resident halo kernel: one workgroup per CU, the column groups side by side, each
// group's blocks over contiguous tile ranges (neighbouring tiles share most of their halo rows in
// the L2).  MATRIX_AMD_CONV_HALO=0 takes the tile kernel instead.
bool halo_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("MATRIX_AMD_CONV_HALO");
        return !(e && e[0] == '0');
    }();
    return on;
}

// The halo geometry of a same convolution, or false when the halo kernel does not apply: one
// group, 2 or more kernel positions and at most 9 K pairs of 64 channels (16-bit) over all of
// them, stride 1 and each output extent equal to its input extent, the halo within a ring half, C
// rows in whole 16-byte units.
template <int NS>
bool halo_geom(const ConvShape& cs, uint32_t Cgp, const int* pad_lo, const int* stride, const int* dil,
               wres::HaloGeom& hg) {
    if (cs.groups != 1 || (Cgp * 2) % (uint32_t)tile::ROWB || cs.out_s[NS + 1] != 1) return false;
    const uint32_t cp = Cgp * 2 / (uint32_t)tile::ROWB;
    uint32_t kpos = 1;
    for (int d = 0; d < NS; d++) {
        if (stride[d] != 1 || cs.OS[d] != cs.S[d]) return false;
        kpos *= cs.K[d];
    }
    // a 1 x 1 kernel reads each pixel once, so a halo saves nothing: the tile kernel's GEMM runs it
    // faster (config 4's 1 x 1 stride-2 product after its pack: 7.0 against 7.8 us)
    if (kpos < 2 || kpos * cp > (uint32_t)wres::MAX_KP) return false;
    for (int a = 0; a <= NS; a++)
        if ((cs.out_s[a] * 2) % 16) return false;
    hg = wres::HaloGeom{};
    const uint32_t S0 = NS == 2 ? cs.S[0] : 1, S1 = cs.S[NS - 1];
    const uint32_t K0 = NS == 2 ? cs.K[0] : 1, K1 = cs.K[NS - 1];
    const int d0 = NS == 2 ? dil[0] : 1, d1 = dil[NS - 1];
    const int p0 = NS == 2 ? pad_lo[0] : 0, p1 = pad_lo[NS - 1];
    int64_t lo = 0, hi = 0;
    for (uint32_t k0 = 0; k0 < K0; k0++)
        for (uint32_t k1 = 0; k1 < K1; k1++) {
            const uint32_t t = k0 * K1 + k1;
            const int64_t a0 = (int64_t)k0 * d0 - p0, a1 = (int64_t)k1 * d1 - p1;
            const int64_t sh = a0 * S1 + a1;
            if (sh < lo) lo = sh;
            if (sh > hi) hi = sh;
            for (uint32_t b = 0; b < cp; b++) {
                hg.dk0[t * cp + b] = (int32_t)a0;
                hg.dk1[t * cp + b] = (int32_t)a1;
                hg.sh[t * cp + b] = (int32_t)(sh * cp + b);
            }
        }
    const int64_t rows = ((wres::BM + (-lo) + hi) * (int64_t)cp + 7) / 8 * 8;
    if (rows > wres::MAX_HALO) return false;
    // the halo must save DMA against gathering each K pair's 64 rows: at 352 halo rows for 384
    // gathered (3 x 1 over 128 channels of 56-pixel rows) the tile kernel ran 18.2 against 19.7 us;
    // at 136 / 384 (1 x 3), 360 / 576 (3 x 1, 192 channels) and 184 / 576 (config 4) the halo kernel
    // ran 17.5 / 14.1 / 21.5 against 18.2 / 18.9 / 23.8 us
    if (4 * rows > 3 * (int64_t)wres::BM * kpos * cp) return false;
    hg.s0 = FastDiv(S0);
    hg.s1 = FastDiv(S1);
    hg.cp = FastDiv(cp);
    hg.rlo = (int32_t)(-lo);
    hg.hrows = (uint32_t)rows;
    hg.npix = (uint32_t)((uint64_t)cs.N * S0 * S1);
    hg.on = (uint32_t)cs.out_s[0];
    hg.os0 = NS == 2 ? (uint32_t)cs.out_s[1] : 0;
    hg.os1 = (uint32_t)cs.out_s[NS];
    return true;
}

template <int DT>
int launch_halo(GemmArgs g, const wres::HaloGeom& hg, void* out, const void* xp, const void* wp, hipStream_t st) {
    const uint32_t kp = g.K / (tile::ROWB / 2);
    g.tiles_m = (g.M + wres::BM - 1) / wres::BM;
    const uint32_t cgs = (g.N + wres::BNC - 1) / wres::BNC;
    uint32_t bpc = cgs >= 256 ? 1 : 256 / cgs;
    if (bpc > g.tiles_m) bpc = g.tiles_m;
    const uint64_t blocks = (uint64_t)cgs * bpc;
    if (blocks > 0x7fffffffull) return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: grid too large");
    auto go = [&](auto kpc) -> int {
        constexpr int KP = decltype(kpc)::value;
        if (hg.cp.d == 1)
            hipLaunchKernelGGL((wres::conv_halo_kernel<DT, KP, true>), dim3((uint32_t)blocks), dim3(512), 0, st,
                               static_cast<uint16_t*>(out), static_cast<const uint16_t*>(xp),
                               static_cast<const uint16_t*>(wp), g, hg, bpc);
        else
            hipLaunchKernelGGL((wres::conv_halo_kernel<DT, KP, false>), dim3((uint32_t)blocks), dim3(512), 0, st,
                               static_cast<uint16_t*>(out), static_cast<const uint16_t*>(xp),
                               static_cast<const uint16_t*>(wp), g, hg, bpc);
        MX_HIP(hipGetLastError());
        return MX_OK;
    };
    switch (kp) {
    case 1: return go(std::integral_constant<int, 1>{});
    case 2: return go(std::integral_constant<int, 2>{});
    case 3: return go(std::integral_constant<int, 3>{});
    case 4: return go(std::integral_constant<int, 4>{});
    case 5: return go(std::integral_constant<int, 5>{});
    case 6: return go(std::integral_constant<int, 6>{});
    case 7: return go(std::integral_constant<int, 7>{});
    case 8: return go(std::integral_constant<int, 8>{});
    case 9: return go(std::integral_constant<int, 9>{});
    default: return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: halo kernel past 9 kernel positions");
    }
}

template <int DT, int NS>
int launch_implicit_gemm(const ConvShape& cs, uint32_t Cgp, const int* pad_lo, const int* stride, const int* dil,
                         void* out, const void* xp, const void* wp, hipStream_t st) {
    using S = typename MmaTraits<DT>::S;
    constexpr uint32_t PE = tile::ROWB / sizeof(S);
    typename ConvSrc<NS>::Geom geo{};
    uint64_t M = cs.N, kpos = 1;
    for (int d = 0; d < NS; d++) {
        geo.odim[d] = FastDiv(cs.OS[d]);
        geo.idim[d] = cs.S[d];
        geo.stride[d] = stride[d];
        geo.dil[d] = dil[d];
        geo.pad[d] = pad_lo[d];
        geo.kdim[d] = FastDiv(cs.K[d]);
        M *= cs.OS[d];
        kpos *= cs.K[d];
    }
    uint32_t xs = cs.groups * Cgp;
    for (int d = NS - 1; d >= 0; --d) {
        geo.xs[d] = xs;
        xs *= cs.S[d];
    }
    geo.xn = xs;
    geo.cpairs = FastDiv(Cgp / PE);
    geo.on = (uint32_t)cs.out_s[0];
    for (int d = 0; d < NS; d++) geo.os[d] = (uint32_t)cs.out_s[d + 1];

    GemmArgs g{};
    g.M = (uint32_t)M;
    g.N = cs.Og;
    g.K = (uint32_t)(kpos * Cgp);
    g.lda = 0;
    g.ka = 1;
    g.ldb = g.K;
    g.kb = 1;
    g.ldc = 0;
    g.cn = (uint32_t)cs.out_s[NS + 1];
    g.batches = cs.groups;
    if (cs.groups > 1) {
        g.bd.n = 1;
        g.bd.shape[0] = FastDiv(cs.groups);
        g.bd.sA[0] = Cgp;
        g.bd.sB[0] = cs.Og * g.K;
        g.bd.sC[0] = (uint32_t)(cs.Og * cs.out_s[NS + 1]);
    }
    if constexpr (DT != MX_FLOAT32) {
        wres::HaloGeom hg;
        if ((uintptr_t)out % 16 == 0 && halo_enabled() && halo_geom<NS>(cs, Cgp, pad_lo, stride, dil, hg))
            return launch_halo<DT>(g, hg, out, xp, wp, st);
    }
    return tile::launch_tile_kernel<DT, true, false, ConvSrc<NS>>(tile::choose_tile(g.M, g.N, g.batches), g, geo,
                                                                  out, xp, wp, st, "mx_launch_conv_nd");
}

template <int DT>
int launch_direct(const ConvShape& cs, const int* pad_lo, const int* stride, const int* dil, const int* dil_lhs,
                  int flip, void* out, const void* in, const void* kern, hipStream_t st) {
    using S = typename dt_traits<DT>::S;
    DirectDesc d{};
    d.ns = cs.ns;
    d.N = cs.N; d.O = cs.O; d.Cg = cs.Cg; d.Og = cs.Og; d.groups = cs.groups;
    uint64_t total = (uint64_t)cs.N * cs.O, kdot = cs.Cg;
    for (int a = 0; a < cs.ns; a++) {
        d.S[a] = cs.S[a]; d.K[a] = cs.K[a]; d.OS[a] = cs.OS[a];
        d.pad[a] = pad_lo[a]; d.stride[a] = stride[a]; d.dil[a] = dil[a]; d.dil_lhs[a] = dil_lhs[a];
        total *= cs.OS[a];
        kdot *= cs.K[a];
    }
    for (int a = 0; a < cs.ns + 2; a++) { d.in_s[a] = cs.in_s[a]; d.k_s[a] = cs.k_s[a]; d.out_s[a] = cs.out_s[a]; }
    d.flip = flip;
    d.kdot = kdot;
    if (total == 0) return MX_OK;
    const uint64_t want = (total + 255) / 256;
    hipLaunchKernelGGL((conv_direct_kernel<DT>), dim3((uint32_t)(want < 1048576 ? want : 1048576)), dim3(256), 0, st,
                       (S*)out, (const S*)in, (const S*)kern, total, d);
    MX_HIP(hipGetLastError());
    return MX_OK;
}

// A 1 x 1 kernel, no padding, one group, a stride above 1, 16-byte aligned packed rows: the
// sampled positions alone are packed (a quarter of the image at stride 2).
bool sampled_1x1(const ConvShape& cs, const int* pad_lo, const int* stride) {
    if (cs.groups != 1 || cs.ns < 1 || cs.ns > 2) return false;
    bool strided = false;
    for (int d = 0; d < cs.ns; d++) {
        if (cs.K[d] != 1 || pad_lo[d] != 0 || stride[d] < 1) return false;
        if ((uint64_t)(cs.OS[d] - 1) * stride[d] >= cs.S[d]) return false;
        strided |= stride[d] > 1;
    }
    return strided;
}

template <int DT>
int launch_mfma_path(const ConvShape& cs, const Plan& p, const int* pad_lo, const int* stride, const int* dil,
                     int flip, void* out, const void* in, const void* kern, void* ws, hipStream_t st) {
    using S = typename MmaTraits<DT>::S;
    char* w = static_cast<char*>(ws);
    const void* xp = in;
    if (p.pack_in && sampled_1x1(cs, pad_lo, stride) && (uintptr_t)w % 16 == 0) {
        // pack the sampled positions only, then a stride-1 product over them
        S* xs = reinterpret_cast<S*>(w);
        constexpr uint32_t VE = 16 / sizeof(S);
        uint32_t OP = 1;
        for (int d = 0; d < cs.ns; d++) OP *= cs.OS[d];
        if (cs.in_s[cs.ns] == 1 && cs.in_s[cs.ns + 1] != 1) {
            // channel-major image (NCHW seen channels-last): load along the spatial axis
            const dim3 grid((OP + 63) / 64, (p.Cgp + 63) / 64, cs.N);
            hipLaunchKernelGGL((pack_input_sampled_cm_kernel<S>), grid, dim3(256), 0, st, xs, static_cast<const S*>(in),
                               OP, FastDiv(cs.OS[cs.ns - 1]), cs.ns, cs.C, p.Cgp, cs.in_s[0], cs.in_s[cs.ns + 1],
                               cs.in_s[1], cs.ns == 2 ? cs.in_s[2] : 0, (uint32_t)stride[0],
                               cs.ns == 2 ? (uint32_t)stride[1] : 0u);
        } else {
            const dim3 grid((OP + 31) / 32, (p.Cgp + 8 * VE - 1) / (8 * VE), cs.N);
            hipLaunchKernelGGL((pack_input_sampled_kernel<S>), grid, dim3(256), 0, st, xs, static_cast<const S*>(in),
                               OP, FastDiv(cs.OS[cs.ns - 1]), cs.ns, cs.C, p.Cgp, cs.in_s[0], cs.in_s[cs.ns + 1],
                               cs.in_s[1], cs.ns == 2 ? cs.in_s[2] : 0, (uint32_t)stride[0],
                               cs.ns == 2 ? (uint32_t)stride[1] : 0u);
        }
        MX_HIP(hipGetLastError());
        const void* wq = kern;
        if (p.pack_k || flip) {
            if (int rc = launch_pack_kernel<S>(cs, p.Cgp, flip, reinterpret_cast<S*>(w + p.xp_bytes),
                                               static_cast<const S*>(kern), st))
                return rc;
            wq = w + p.xp_bytes;
        }
        ConvShape cd = cs;
        for (int d = 0; d < cs.ns; d++) cd.S[d] = cs.OS[d];
        const int one[kMaxSpatial] = {1, 1, 1, 1, 1, 1}, zero[kMaxSpatial] = {};
        if (cs.ns == 1) return launch_implicit_gemm<DT, 1>(cd, p.Cgp, zero, one, one, out, xs, wq, st);
        return launch_implicit_gemm<DT, 2>(cd, p.Cgp, zero, one, one, out, xs, wq, st);
    }
    if (p.pack_in && (p.pack_k || flip)) {
        // both packs in one launch when the input takes the 16-byte transpose
        S* xs = reinterpret_cast<S*>(w);
        S* wsp = reinterpret_cast<S*>(w + p.xp_bytes);
        uint64_t P;
        dim3 grid;
        if (transpose16_grid(cs, p.Cgp, xs, static_cast<const S*>(in), &grid, &P)) {
            PackKDesc d;
            uint64_t wtotal;
            if (int rc = pack_kernel_desc(cs, p.Cgp, flip, d, wtotal)) return rc;
            const uint64_t nwb = (wtotal + 255) / 256;
            const uint64_t blocks = nwb + (uint64_t)grid.x * grid.y * grid.z;
            if (blocks > 0x7fffffffull) return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: pack grid too large");
            hipLaunchKernelGGL((pack_input16_and_kernel_kernel<S>), dim3((uint32_t)blocks), dim3(256), 0, st, xs,
                               static_cast<const S*>(in), (uint32_t)P, cs.C, p.Cgp, cs.in_s[0], cs.in_s[cs.ns + 1],
                               grid.x, grid.y, wsp, static_cast<const S*>(kern), (uint32_t)wtotal, (uint32_t)nwb, d);
            MX_HIP(hipGetLastError());
            if (cs.ns == 1) return launch_implicit_gemm<DT, 1>(cs, p.Cgp, pad_lo, stride, dil, out, xs, wsp, st);
            return launch_implicit_gemm<DT, 2>(cs, p.Cgp, pad_lo, stride, dil, out, xs, wsp, st);
        }
    }
    if (p.pack_in) {
        int rc = launch_pack_input<S>(cs, p.Cgp, reinterpret_cast<S*>(w), static_cast<const S*>(in), st);
        if (rc) return rc;
        xp = w;
        w += p.xp_bytes;
    }
    const void* wp = kern;
    if (p.pack_k || flip) {
        int rc = launch_pack_kernel<S>(cs, p.Cgp, flip, reinterpret_cast<S*>(w), static_cast<const S*>(kern), st);
        if (rc) return rc;
        wp = w;
    }
    if (cs.ns == 1) return launch_implicit_gemm<DT, 1>(cs, p.Cgp, pad_lo, stride, dil, out, xp, wp, st);
    return launch_implicit_gemm<DT, 2>(cs, p.Cgp, pad_lo, stride, dil, out, xp, wp, st);
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_conv_workspace_bytes(int dtype, int nspatial, const uint32_t* in_shape, const uint32_t* k_shape,
                                       const uint32_t* out_shape, const uint32_t* in_strides,
                                       const uint32_t* k_strides, const uint32_t* out_strides, int groups,
                                       size_t* bytes) {
    if (!bytes) return fail(MX_ERR_INVALID_ARG, "mx_conv_workspace_bytes: null result pointer");
    *bytes = 0;
    ConvShape cs{};
    int rc = read_shape(dtype, nspatial, in_shape, k_shape, out_shape, in_strides, k_strides, out_strides, groups, cs,
                        "mx_conv_workspace_bytes");
    if (rc) return rc;
    const Plan p = plan_conv(dtype, cs);
    if (p.mfma) *bytes = p.xp_bytes + p.wp_bytes;
    return MX_OK;
}

extern "C" int mx_launch_conv_nd(int dtype, int nspatial, const uint32_t* in_shape, const uint32_t* k_shape,
                                 const uint32_t* out_shape, const uint32_t* in_strides, const uint32_t* k_strides,
                                 const uint32_t* out_strides, const int* pad_lo, const int* stride,
                                 const int* dil_rhs, const int* dil_lhs, int groups, int flip, void* out,
                                 const void* in, const void* kern, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    ConvShape cs{};
    int rc = read_shape(dtype, nspatial, in_shape, k_shape, out_shape, in_strides, k_strides, out_strides, groups, cs,
                        "mx_launch_conv_nd");
    if (rc) return rc;
    if (!pad_lo || !stride || !dil_rhs || !dil_lhs) return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: null geometry");
    bool no_lhs_dil = true;
    for (int d = 0; d < nspatial; d++) {
        if (stride[d] < 1 || dil_rhs[d] < 1 || dil_lhs[d] < 1)
            return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: stride and dilations must be >= 1");
        no_lhs_dil = no_lhs_dil && dil_lhs[d] == 1;
    }
    uint64_t total = (uint64_t)cs.N * cs.O;
    for (int d = 0; d < nspatial; d++) total *= cs.OS[d];
    if (total == 0) return MX_OK;
    if (!out || !in || !kern) return fail(MX_ERR_INVALID_ARG, "mx_launch_conv_nd: null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;

    const Plan p = plan_conv(dtype, cs);
    bool spatial_ok = true;                           // strided positions fit the 16-bit packing
    for (int d = 0; d < nspatial && p.mfma; d++)
        spatial_ok = spatial_ok && (uint64_t)(cs.OS[d] ? cs.OS[d] - 1 : 0) * stride[d] < 32768 &&
                     (uint64_t)pad_lo[d] < 32768 && (uint64_t)(cs.K[d] - 1) * dil_rhs[d] < 32768;
    if (p.mfma && no_lhs_dil && spatial_ok) {
        const size_t need = p.xp_bytes + p.wp_bytes;
        const bool aligned = (p.pack_in || (uintptr_t)in % 16 == 0) && (p.pack_k || flip || (uintptr_t)kern % 16 == 0) &&
                             ((uintptr_t)workspace % 16 == 0);
        if (workspace_bytes < need || (!workspace && need))
            return fail(MX_ERR_WORKSPACE, "mx_launch_conv_nd: workspace of " + std::to_string(need) +
                                              " bytes required (mx_conv_workspace_bytes)");
        if (aligned) {
            switch (dtype) {
            case MX_FLOAT32: return launch_mfma_path<MX_FLOAT32>(cs, p, pad_lo, stride, dil_rhs, flip, out, in, kern, workspace, st);
            case MX_FLOAT16: return launch_mfma_path<MX_FLOAT16>(cs, p, pad_lo, stride, dil_rhs, flip, out, in, kern, workspace, st);
            case MX_BFLOAT16: return launch_mfma_path<MX_BFLOAT16>(cs, p, pad_lo, stride, dil_rhs, flip, out, in, kern, workspace, st);
            default: break;
            }
        }
    }
    switch (dtype) {
    case MX_FLOAT32: return launch_direct<MX_FLOAT32>(cs, pad_lo, stride, dil_rhs, dil_lhs, flip, out, in, kern, st);
    case MX_FLOAT16: return launch_direct<MX_FLOAT16>(cs, pad_lo, stride, dil_rhs, dil_lhs, flip, out, in, kern, st);
    case MX_BFLOAT16: return launch_direct<MX_BFLOAT16>(cs, pad_lo, stride, dil_rhs, dil_lhs, flip, out, in, kern, st);
    case MX_INT32: return launch_direct<MX_INT32>(cs, pad_lo, stride, dil_rhs, dil_lhs, flip, out, in, kern, st);
    case MX_INT64: return launch_direct<MX_INT64>(cs, pad_lo, stride, dil_rhs, dil_lhs, flip, out, in, kern, st);
    default:
        return fail(MX_ERR_UNSUPPORTED, "mx_launch_conv_nd: no kernel for dtype " + std::to_string(dtype));
    }
}
