// reduce_plans.hpp -- the reduction plans shared by the single-op kernels (reduce.hip) and the
// group kernels (reduce_group.hip).
//
// Semantics follow the reference CPU backends (Matrix.mm:15099-15208 sum,
// Matrix.mm:14812-15059 max / min, Matrix.mm:16182-16458 argmax / argmin):
//   - Max / Min start from dtype_lowest / dtype_max (matrix.h:271-282) and replace the
//     running value only when strictly better, so NaN never wins, an all -inf row gives
//     -FLT_MAX, and among equal values (+0 / -0) the first index wins;
//   - ArgMax / ArgMin give the first index of the extremum as int32, 0 when nothing is
//     strictly better than the start value;
//   - integer sums wrap in the element type; 16-bit float sums accumulate in fp32.
// Every partial carries the index it came from and the combine step breaks value ties by
// the smaller index, so any split of the axis over lanes, waves and blocks reproduces the
// sequential left-to-right result bit for bit.  fp32 sums are a fixed-shape tree
// (deterministic run to run, within tolerance of the sequential sum).
//
// Plans, chosen on the host from the CollapsedDims_2 descriptor:
//   lane   reduce stride 1, rows of at most four 128-bit vectors: one lane per output, every
//          load of the row issued before the first compare;
//   rows   reduce stride 1, medium rows: L lanes per output (L = 4, 16, 64), 128-bit loads,
//          several outputs in flight per lane group;
//   block  reduce stride 1, long rows: a 1024- or 256-thread block per output (or per chunk);
//   short  reduce stride != 1, at most 8 reduced elements: a lane owns VEC consecutive outputs
//          and issues all of their loads at once;
//   cols   reduce stride != 1, longer axes: a lane owns VEC consecutive outputs, the four waves
//          of a block split the reduced axis between them and combine through LDS.
// Loads in flight per lane are kept moderate (4-8 vectors): on this part a 64 MiB read is
// fastest with about 1-4 KiB in flight per wave; more queued requests per CU slow it down.
// The plans avoid splitting one output's axis over blocks whenever the outputs alone cover the
// CUs; when they must split, each block writes its partial to the workspace and a second launch
// combines the partials in split order.
#pragma once
#include "reduce_ops.hpp"

namespace mx {

// A reduction's collapsed descriptor (CollapsedDims_2 plus the reduced axis' stride and extent).
struct Desc {
    int cd;
    uint32_t shape[MX_MAX_DIMS], so[MX_MAX_DIMS], si[MX_MAX_DIMS];
    uint32_t rs, n;
};

namespace {

// ------------------------------------------------------------------ descriptors
// Input offset of output g: the reference decomposes g with the collapsed output strides
// (off = sum_i (rem / sOut_i) * sIn_i; rem %= sOut_i), Matrix.mm:15190-15194.
struct OffDesc {
    int n;
    FastDiv so[MX_MAX_DIMS];
    uint32_t si[MX_MAX_DIMS];
    __device__ __forceinline__ uint64_t offset(uint32_t g) const {
        uint64_t off = 0;
        uint32_t rem = g;
        for (int i = 0; i < n; i++) {
            uint32_t q = so[i].div(rem);
            off += (uint64_t)q * si[i];
            rem -= q * so[i].d;
        }
        return off;
    }
};

template <typename S, int VEC>
struct alignas(VEC * sizeof(S) >= 16 ? 16 : VEC * sizeof(S)) VecT { S v[VEC]; };

// The coalesced plans read their input with ld_stream (nontemporal loads, common.hpp): the axis-1
// and axis-0 reductions of a [256, 65536] f32 input rise from 5.80 to 6.24 TB/s and from 5.74 to
// 6.40 TB/s.  The gapped lane plan keeps ordinary loads: each lane's row is split over several load
// instructions that share lines, and nontemporal loads there fell from 5.37 to 3.43 TB/s.

// Partials of a split axis are combined by reduce_finalize_kernel, a second launch on the same
// stream.  (Combining them inside the first launch needs a device-scope release per block; on
// this multi-XCD part that is an L2 write-back, which costs more than the extra launch.)

// Every plan is a device function (the *_body templates) taking its block coordinates and, where
// it combines waves, an LDS buffer; a single-op kernel and a group kernel wrap it.  A group
// kernel runs several reductions of one dtype over one descriptor in one launch: blockIdx.z picks
// the member, whose op, input, output and partials come from GroupPtrs (see run_reduce_group).
constexpr int kGroupMax = 8;
struct GroupPtrs {
    int op[kGroupMax];
    const void* in[kGroupMax];
    void* out[kGroupMax];
    void* part[kGroupMax];
};

// Largest reduction state of a dtype over the five ops (sizes the group kernels' LDS).
template <int DT>
constexpr size_t kMaxState = sizeof(typename RedSel<DT, MX_RED_ARGMAX>::R::St) > sizeof(typename RedSel<DT, MX_RED_SUM>::R::St)
                                 ? sizeof(typename RedSel<DT, MX_RED_ARGMAX>::R::St)
                                 : sizeof(typename RedSel<DT, MX_RED_SUM>::R::St);

// Calls f(integral_constant<op>) for a runtime op (uniform over the block).
template <typename F>
__device__ __forceinline__ void op_switch(int op, F&& f) {
    switch (op) {
    case MX_RED_SUM: f(std::integral_constant<int, MX_RED_SUM>{}); break;
    case MX_RED_MAX: f(std::integral_constant<int, MX_RED_MAX>{}); break;
    case MX_RED_MIN: f(std::integral_constant<int, MX_RED_MIN>{}); break;
    case MX_RED_ARGMAX: f(std::integral_constant<int, MX_RED_ARGMAX>{}); break;
    default: f(std::integral_constant<int, MX_RED_ARGMIN>{}); break;
    }
}

template <int DT, int OP> using OutOf = typename RedSel<DT, OP>::R::OutT;
template <int DT, int OP> using StOf = typename RedSel<DT, OP>::R::St;
template <int DT> using ElemOf = typename dt_traits<DT>::S;

// ------------------------------------------------------------------ rows (stride 1), L lanes per output
// U outputs per lane group are in flight at once; every group runs the same number of rounds so
// the group shuffles always see all of their lanes active.
template <int DT, int OP, int VEC, int L, int U>
__device__ __forceinline__ void rows_body(OutOf<DT, OP>* __restrict__ out, const ElemOf<DT>* __restrict__ in,
                                          uint32_t total_out, uint32_t n, uint32_t rounds, const OffDesc& od,
                                          uint32_t bx, uint32_t gx) {
    using R = typename RedSel<DT, OP>::R;
    using S = ElemOf<DT>;
    using V = VecT<S, VEC>;
    using St = typename R::St;
    constexpr int GPB = 256 / L;                         // groups per block
    constexpr bool NT = L * sizeof(V) >= 128;            // a group's load covers whole lines
    const uint32_t group = bx * GPB + threadIdx.x / L;
    const uint32_t lane = threadIdx.x % L;
    const uint32_t ngroups = gx * GPB;
    for (uint32_t r = 0; r < rounds; r++) {
        St st[U];
        const S* row[U];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            uint64_t g = (uint64_t)(r * U + u) * ngroups + group;
            valid[u] = g < total_out;
            row[u] = in + (valid[u] ? od.offset((uint32_t)g) : 0);
            st[u] = R::init();
        }
#pragma unroll 4
        for (uint32_t e = lane * VEC; e < n; e += L * VEC) {
            V v[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                if (valid[u]) {
                    const V* p = reinterpret_cast<const V*>(row[u] + e);
                    v[u] = NT ? ld_stream(p) : *p;
                }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (valid[u]) {
#pragma unroll
                    for (int k = 0; k < VEC; k++) R::step(st[u], v[u].v[k], e + k);
                }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int m = L / 2; m >= 1; m >>= 1) st[u] = R::combine(st[u], R::shfl(st[u], m));
            uint64_t g = (uint64_t)(r * U + u) * ngroups + group;
            if (valid[u] && lane == 0) out[g] = R::out(st[u]);
        }
    }
}


// ------------------------------------------------------------------ lane (stride 1, rows of <= 4 vectors)
// One lane per output; the nv <= NV vectors of the row are all loaded before any is used.
template <int DT, int OP, int VEC, int NV>
__device__ __forceinline__ void lane_body(OutOf<DT, OP>* __restrict__ out, const ElemOf<DT>* __restrict__ in,
                                          uint32_t total_out, uint32_t nv, const OffDesc& od, uint32_t bx) {
    using R = typename RedSel<DT, OP>::R;
    using S = ElemOf<DT>;
    using V = VecT<S, VEC>;
    const uint32_t g = bx * 256 + threadIdx.x;
    if (g >= total_out) return;
    const S* row = in + od.offset(g);
    V v[NV];
#pragma unroll
    for (int u = 0; u < NV; u++)
        if (u < nv) v[u] = *reinterpret_cast<const V*>(row + u * VEC);
    typename R::St st = R::init();
#pragma unroll
    for (int u = 0; u < NV; u++)
        if (u < nv) {
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st, v[u].v[k], u * VEC + k);
        }
    out[g] = R::out(st);
}

// ------------------------------------------------------------------ lane, packed rows
// Rows of nv <= 4 vectors stored back to back (input offset of output g is g * n): a block's 256
// rows are one run of 256 * nv vectors.  It is read with whole-line streaming loads (vector f of
// the run by thread f % 256), staged in LDS, and each lane then reduces its own row from LDS in the
// order of lane_body, so both give the same bits.  LDS position of vector f: f ^ ((f >> 4) & mask)
// with mask 3 for nv = 4 and 1 for nv = 2, which moves the chunks within their row so the 16 lanes
// of one 128-bit LDS read pass hit distinct banks (nv = 3 and 1 need no swizzle).
// smem: 1024 vectors (16 KiB).
template <int DT, int OP, int VEC>
__device__ __forceinline__ void lane_packed_body(OutOf<DT, OP>* __restrict__ out, const ElemOf<DT>* __restrict__ in,
                                                 uint32_t total_out, uint32_t nv, uint32_t bx, void* smem) {
    using R = typename RedSel<DT, OP>::R;
    using S = ElemOf<DT>;
    using V = VecT<S, VEC>;
    V* sh = static_cast<V*>(smem);
    const uint32_t g0 = bx * 256;
    const uint32_t rows = min(256u, total_out - g0);
    const uint32_t nvec = rows * nv;
    const uint32_t mask = nv == 4 ? 3u : nv == 2 ? 1u : 0u;
    const V* src = reinterpret_cast<const V*>(in) + (uint64_t)g0 * nv;
    const uint32_t t = threadIdx.x;
    V v[4];
#pragma unroll
    for (int w = 0; w < 4; w++)
        if (t + 256u * w < nvec) v[w] = ld_stream(src + t + 256u * w);
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t f = t + 256u * w;
        if (f < nvec) sh[f ^ ((f >> 4) & mask)] = v[w];
    }
    __syncthreads();
    if (t >= rows) return;
    typename R::St st = R::init();
#pragma unroll
    for (int u = 0; u < 4; u++)
        if (u < (int)nv) {
            const uint32_t f = t * nv + u;
            const V x = sh[f ^ ((f >> 4) & mask)];
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st, x.v[k], u * VEC + k);
        }
    out[g0 + t] = R::out(st);
}


// ------------------------------------------------------------------ block (stride 1, long rows)
// One block of 64 * WAVES threads per (output g, chunk c).  U vectors per lane are in flight; the
// last partial round issues its loads together.  smem: WAVES states.
template <int DT, int OP, int VEC, int WAVES, int U>
__device__ __forceinline__ void block_body(OutOf<DT, OP>* __restrict__ out, StOf<DT, OP>* __restrict__ part,
                                           const ElemOf<DT>* __restrict__ in, uint32_t total_out, uint32_t n,
                                           uint32_t chunk, uint32_t nsplit, const OffDesc& od, uint32_t g, uint32_t c,
                                           void* smem) {
    using R = typename RedSel<DT, OP>::R;
    using S = ElemOf<DT>;
    using V = VecT<S, VEC>;
    using St = typename R::St;
    constexpr uint32_t STEP = 64 * WAVES * VEC;
    const uint32_t beg = c * chunk;
    const uint32_t end = min(n, beg + chunk);
    const S* row = in + od.offset(g);
    St st = R::init();
    uint32_t e = beg + threadIdx.x * VEC;
    for (; e + (U - 1) * STEP < end; e += U * STEP) {
        V v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = ld_stream(reinterpret_cast<const V*>(row + e + u * STEP));
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st, v[u].v[k], e + u * STEP + k);
    }
    if constexpr (U > 1) if (e < end) {
        V v[U - 1];
#pragma unroll
        for (int u = 0; u < U - 1; u++)
            if (e + u * STEP < end) v[u] = ld_stream(reinterpret_cast<const V*>(row + e + u * STEP));
#pragma unroll
        for (int u = 0; u < U - 1; u++)
            if (e + u * STEP < end) {
#pragma unroll
                for (int k = 0; k < VEC; k++) R::step(st, v[u].v[k], e + u * STEP + k);
            }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) st = R::combine(st, R::shfl(st, m));
    St* wpart = static_cast<St*>(smem);
    if ((threadIdx.x & 63) == 0) wpart[threadIdx.x >> 6] = st;
    __syncthreads();
    St r = wpart[0];
#pragma unroll
    for (int w = 1; w < WAVES; w++) r = R::combine(r, wpart[w]);
    if (threadIdx.x == 0) {
        if (nsplit == 1) out[g] = R::out(r);
        else part[(uint64_t)c * total_out + g] = r;
    }
}


// ------------------------------------------------------------------ cols (stride != 1)
// Lane l of every wave owns outputs [(bx * 64 + l) * VEC, +VEC); the WAVES waves of the block take
// interleaved rows of the block's share [c * chunk, ...) of the reduced axis.  smem: (WAVES - 1) x
// 64 VEC states.
template <int DT, int OP, int VEC, int WAVES>
__device__ __forceinline__ void cols_body(OutOf<DT, OP>* __restrict__ out, StOf<DT, OP>* __restrict__ part,
                                          const ElemOf<DT>* __restrict__ in, uint32_t total_out, uint32_t n, uint32_t rs,
                                          uint32_t chunk, uint32_t nsplit, const OffDesc& od, uint32_t bx, uint32_t c,
                                          void* smem) {
    using R = typename RedSel<DT, OP>::R;
    using S = ElemOf<DT>;
    using V = VecT<S, VEC>;
    using St = typename R::St;
    constexpr int U = 8;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t g0 = (bx * 64 + lane) * VEC;
    const bool valid = g0 < total_out;
    const uint32_t beg = c * chunk;
    const uint32_t end = min(n, beg + chunk);
    const S* base = in + (valid ? od.offset(g0) : 0);
    St st[VEC];
#pragma unroll
    for (int k = 0; k < VEC; k++) st[k] = R::init();
    if (valid) {
        uint32_t i = beg + wave;
        for (; i + (U - 1) * WAVES < end; i += U * WAVES) {
            V v[U];
#pragma unroll
            for (int u = 0; u < U; u++) v[u] = ld_stream(reinterpret_cast<const V*>(base + (uint64_t)(i + u * WAVES) * rs));
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int k = 0; k < VEC; k++) R::step(st[k], v[u].v[k], i + u * WAVES);
        }
        if (i < end) {
            V v[U - 1];
#pragma unroll
            for (int u = 0; u < U - 1; u++)
                if (i + u * WAVES < end) v[u] = ld_stream(reinterpret_cast<const V*>(base + (uint64_t)(i + u * WAVES) * rs));
#pragma unroll
            for (int u = 0; u < U - 1; u++)
                if (i + u * WAVES < end) {
#pragma unroll
                    for (int k = 0; k < VEC; k++) R::step(st[k], v[u].v[k], i + u * WAVES);
                }
        }
    }
    // combine the waves' states through LDS, in wave order
    if constexpr (WAVES > 1) {
        St* sh = static_cast<St*>(smem);                 // [WAVES - 1][64 VEC]
        if (wave > 0) {
#pragma unroll
            for (int k = 0; k < VEC; k++) sh[(wave - 1) * 64 * VEC + lane * VEC + k] = st[k];
        }
        __syncthreads();
        if (wave == 0) {
            for (int w = 0; w < WAVES - 1; w++)
#pragma unroll
                for (int k = 0; k < VEC; k++) st[k] = R::combine(st[k], sh[w * 64 * VEC + lane * VEC + k]);
        }
    }
    if (wave == 0 && valid) {
#pragma unroll
        for (int k = 0; k < VEC; k++) {
            if (nsplit == 1) out[g0 + k] = R::out(st[k]);
            else part[(uint64_t)c * total_out + g0 + k] = st[k];
        }
    }
}


// ------------------------------------------------------------------ short (stride != 1, n <= 8)
// Lane l of wave w owns outputs [((bx * WAVES + w) * 64 + l) * VEC, +VEC) and loads all n <= NMAX of
// their rows at once.  VST: the output is 16-byte aligned and VEC outputs make 16 bytes, so they
// go out in one store.
template <int DT, int OP, int VEC, int NMAX, int WAVES, bool VST>
__device__ __forceinline__ void short_body(OutOf<DT, OP>* __restrict__ out, const ElemOf<DT>* __restrict__ in,
                                           uint32_t total_out, uint32_t n, uint32_t rs, const OffDesc& od, uint32_t bx) {
    using R = typename RedSel<DT, OP>::R;
    using S = ElemOf<DT>;
    using V = VecT<S, VEC>;
    using OutT = typename R::OutT;
    const uint32_t g0 = ((bx * WAVES + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63)) * VEC;
    if (g0 >= total_out) return;
    const S* base = in + od.offset(g0);
    V v[NMAX];
#pragma unroll
    for (int u = 0; u < NMAX; u++)
        if (u < n) v[u] = ld_stream(reinterpret_cast<const V*>(base + (uint64_t)u * rs));
    typename R::St st[VEC];
#pragma unroll
    for (int k = 0; k < VEC; k++) st[k] = R::init();
#pragma unroll
    for (int u = 0; u < NMAX; u++)
        if (u < n) {
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st[k], v[u].v[k], u);
        }
    if constexpr (VST) {
        VecT<OutT, VEC> o;
#pragma unroll
        for (int k = 0; k < VEC; k++) o.v[k] = R::out(st[k]);
        *reinterpret_cast<VecT<OutT, VEC>*>(out + g0) = o;
    } else {
#pragma unroll
        for (int k = 0; k < VEC; k++) out[g0 + k] = R::out(st[k]);
    }
}


// finalize: output g combines its nsplit partials in split order.
template <int DT, int OP>
__device__ __forceinline__ void finalize_body(OutOf<DT, OP>* __restrict__ out, const StOf<DT, OP>* __restrict__ part,
                                              uint32_t total_out, uint32_t nsplit, uint32_t bx) {
    using R = typename RedSel<DT, OP>::R;
    const uint32_t g = bx * 256 + threadIdx.x;
    if (g >= total_out) return;
    typename R::St a = part[g];
    for (uint32_t s = 1; s < nsplit; s++) a = R::combine(a, part[(uint64_t)s * total_out + g]);
    out[g] = R::out(a);
}


// finalize for many partials per output: one 256-thread block per output, a fixed-shape tree.
// smem: 4 states.
template <int DT, int OP>
__device__ __forceinline__ void finalize_wide_body(OutOf<DT, OP>* __restrict__ out,
                                                   const StOf<DT, OP>* __restrict__ part, uint32_t total_out,
                                                   uint32_t nsplit, uint32_t g, void* smem) {
    using R = typename RedSel<DT, OP>::R;
    using St = typename R::St;
    St a = R::init();
    for (uint32_t s = threadIdx.x; s < nsplit; s += 256) a = R::combine(a, part[(uint64_t)s * total_out + g]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) a = R::combine(a, R::shfl(a, m));
    St* w = static_cast<St*>(smem);
    if ((threadIdx.x & 63) == 0) w[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) out[g] = R::out(R::combine(R::combine(w[0], w[1]), R::combine(w[2], w[3])));
}

// ------------------------------------------------------------------ planning
enum Mode { kRows = 0, kBlockMode = 1, kCols = 2, kLane = 3, kShort = 4 };


struct Plan {
    Mode mode = kCols;
    int vec = 1;            // elements per 128-bit load actually used (1 = scalar loads)
    int lanes = 1;          // rows plan: lanes per output
    int unroll = 1;         // rows plan: outputs in flight per lane group
    int waves = 1;          // cols / block / short plans: waves per block
    uint32_t nv = 0;        // lane plan: vectors per row
    bool packed = false;    // lane plan: rows back to back (offset of output g is g * n), vector loads
    uint32_t blocks = 0;    // rows plan: grid size; cols plan: column groups
    uint32_t rounds = 0;
    uint32_t nsplit = 1;    // blocks sharing one output's axis
    uint32_t chunk = 0;     // axis elements per split
    uint32_t total_out = 0;
    size_t state_bytes = 0;
    size_t ws_bytes() const { return nsplit > 1 ? (size_t)nsplit * total_out * state_bytes : 0; }
};

constexpr uint32_t kTargetBlocks = 2048;     // 8 resident 256-thread blocks per CU on 256 CUs

// The split layout depends only on the descriptor (never on pointer alignment), so the
// workspace size reported ahead of time always covers the launch.
Plan make_plan(const Desc& d, size_t elem, size_t stbytes, uintptr_t in_ptr) {
    Plan p;
    uint64_t tot = 1;
    for (int i = 0; i < d.cd; i++) tot *= d.shape[i];
    p.total_out = (uint32_t)tot;
    p.state_bytes = stbytes;
    const int VEC = (int)(16 / elem);
    const bool aligned = in_ptr % 16 == 0;
    if (tot == 0) return p;
    // at most 64 KiB of input: one launch (a split would add a combine launch for microseconds
    // of work)
    const bool small = tot * d.n * elem <= 65536;
    if (d.rs == 1 && d.n > 1) {
        bool v_ok = VEC > 1 && d.n % VEC == 0;
        for (int i = 0; v_ok && i < d.cd; i++) if (d.si[i] % VEC) v_ok = false;
        const uint32_t nominal = v_ok ? (uint32_t)VEC : 1u;
        p.vec = (v_ok && aligned) ? VEC : 1;
        const uint32_t nv = (d.n + nominal - 1) / nominal;
        if (nv <= 4) {
            p.mode = kLane;
            p.nv = p.vec == VEC ? nv : d.n;     // unaligned input: scalar loads (n <= 4 * VEC)
            if (p.nv > 4) p.mode = kRows;       // unaligned and n > 4: the rows plan below
        }
        if (p.mode == kLane) {
            p.blocks = (uint32_t)((tot + 255) / 256);
            p.packed = p.vec == VEC && d.so[d.cd - 1] == 1;
            for (int i = 0; p.packed && i < d.cd; i++)
                if ((uint64_t)d.si[i] != (uint64_t)d.n * d.so[i]) p.packed = false;
        } else if (nv > 1024) {
            // One block per output when there are enough outputs to cover the CUs (no partials,
            // no cross-block step); otherwise split each row into chunks of >= 4 vectors a thread.
            p.mode = kBlockMode;
            p.waves = nv >= 8192 ? 16 : 4;
            const uint64_t threads = 64ull * p.waves;
            const uint64_t want_blocks = p.waves == 16 ? 256 : 1024;
            uint64_t want = (want_blocks + tot - 1) / tot;
            uint64_t maxc = (nv + threads * 4 - 1) / (threads * 4);
            uint64_t nc = want < maxc ? want : maxc;
            if (nc < 1 || small) nc = 1;
            uint32_t chunk_v = (uint32_t)((nv + nc - 1) / nc);
            p.chunk = chunk_v * nominal;
            p.nsplit = (d.n + p.chunk - 1) / p.chunk;
        } else {
            p.mode = kRows;
            p.lanes = nv <= 2 ? 1 : nv <= 16 ? 4 : nv <= 64 ? 16 : 64;
            p.unroll = p.lanes == 64 ? 1 : 4;
            const uint64_t groups_needed = (tot + p.unroll - 1) / p.unroll;
            const uint64_t gpb = 256 / p.lanes;
            uint64_t blocks = (groups_needed + gpb - 1) / gpb;
            if (blocks > 8 * kTargetBlocks) blocks = 8 * kTargetBlocks;
            p.blocks = (uint32_t)blocks;
            const uint64_t per_round = blocks * gpb * p.unroll;
            p.rounds = (uint32_t)((tot + per_round - 1) / per_round);
        }
        return p;
    }
    // column / general
    const int last = d.cd - 1;
    bool v_ok = VEC > 1 && d.so[last] == 1 && d.si[last] == 1 && d.shape[last] % VEC == 0 &&
                d.rs % VEC == 0;
    for (int i = 0; v_ok && i < last; i++) if (d.si[i] % VEC || d.so[i] % VEC) v_ok = false;
    const uint32_t nominal = v_ok ? (uint32_t)VEC : 1u;
    p.vec = (v_ok && aligned) ? VEC : 1;
    const uint64_t groups = (tot + 64ull * nominal - 1) / (64ull * nominal);   // 64-lane column groups
    p.blocks = (uint32_t)groups;
    if (d.n <= 8) {
        // every row load of a lane in flight at once; one wave per block while the groups alone
        // give every CU several waves, else four
        p.mode = kShort;
        p.waves = groups >= 4096 ? 1 : 4;
        p.chunk = d.n;
        return p;
    }
    p.mode = kCols;
    p.waves = 4;
    // split the axis over blocks when there are fewer column groups than CUs
    p.nsplit = 1;
    if (groups < 256 && d.n >= 256 && !small) {
        uint64_t want = (512 + groups - 1) / groups;
        uint64_t maxc = d.n / 128;                 // keep >= 128 axis elements per split
        if (maxc > 4096) maxc = 4096;
        uint64_t nc = want < maxc ? want : maxc;
        if (nc > 1) {
            p.chunk = (uint32_t)((d.n + nc - 1) / nc);
            p.nsplit = (d.n + p.chunk - 1) / p.chunk;
        }
    }
    if (p.nsplit == 1) p.chunk = d.n;
    return p;
}

int check_desc(const char* who, int op, int cdims, const uint32_t* shape, const uint32_t* sOut,
               const uint32_t* sIn, uint32_t rs, uint32_t n, Desc* d) {
    if (op < MX_RED_SUM || op > MX_RED_ARGMIN)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": unknown op " + std::to_string(op));
    if (cdims < 0 || cdims > MX_MAX_DIMS)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": cdims outside [0, 8]");
    if (cdims > 0 && (!shape || !sOut || !sIn))
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null descriptor");
    d->rs = rs;
    d->n = n;
    if (cdims == 0) {   // one output with unit strides, as Matrix.mm:15133-15138
        d->cd = 1; d->shape[0] = 1; d->so[0] = 1; d->si[0] = 1;
        return MX_OK;
    }
    d->cd = cdims;
    uint64_t tot = 1;
    for (int i = 0; i < cdims; i++) {
        d->shape[i] = shape[i]; d->so[i] = sOut[i]; d->si[i] = sIn[i];
        if (sOut[i] == 0) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": zero output stride");
        tot *= shape[i];
    }
    if (tot > 0xffffffffull) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": more than 2^32-1 outputs");
    return MX_OK;
}

template <typename F>
bool dispatch_op(int op, F&& f) {
    switch (op) {
    case MX_RED_SUM: f(std::integral_constant<int, MX_RED_SUM>{}); return true;
    case MX_RED_MAX: f(std::integral_constant<int, MX_RED_MAX>{}); return true;
    case MX_RED_MIN: f(std::integral_constant<int, MX_RED_MIN>{}); return true;
    case MX_RED_ARGMAX: f(std::integral_constant<int, MX_RED_ARGMAX>{}); return true;
    case MX_RED_ARGMIN: f(std::integral_constant<int, MX_RED_ARGMIN>{}); return true;
    default: return false;
    }
}


}  // namespace
}  // namespace mx
