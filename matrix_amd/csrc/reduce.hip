// reduce.hip -- Sum / Max / Min / ArgMax / ArgMin over one axis.
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
// sequential left-to-right result bit for bit.  fp32 sums are a tree (within tolerance).
//
// Plans (chosen on the host from the CollapsedDims_2 descriptor):
//   rows    reduce stride 1: L lanes per output (L = 1, 4, 16, 64) with 128-bit loads;
//   block   reduce stride 1, long rows: one 256-thread block per (output, chunk), chunks
//           combined by a second pass (finalize);
//   cols    reduce stride != 1: a thread owns VEC consecutive outputs and walks the axis,
//           optionally split into chunks combined by finalize.
#include "common.hpp"

#include <climits>
#include <cfloat>
#include <limits>

namespace mx {
namespace {

constexpr int kBlock = 256;
constexpr uint32_t kEmpty = 0x7fffffffu;   // index of a partial that took no element

// ------------------------------------------------------------------ reduction states
template <typename T> __device__ __forceinline__ T shfl_x(T v, int m) { return __shfl_xor(v, m); }
template <> __device__ __forceinline__ uint8_t shfl_x(uint8_t v, int m) { return (uint8_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ int8_t shfl_x(int8_t v, int m) { return (int8_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ uint16_t shfl_x(uint16_t v, int m) { return (uint16_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ int16_t shfl_x(int16_t v, int m) { return (int16_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ uint32_t shfl_x(uint32_t v, int m) { return (uint32_t)__shfl_xor((int)v, m); }
template <> __device__ __forceinline__ uint64_t shfl_x(uint64_t v, int m) { return (uint64_t)__shfl_xor((long long)v, m); }
template <> __device__ __forceinline__ int64_t shfl_x(int64_t v, int m) { return (int64_t)__shfl_xor((long long)v, m); }

template <int DT> struct Limits {
    using C = typename dt_traits<DT>::C;
    __device__ __forceinline__ static C lowest() {
        if constexpr (DT == MX_FLOAT32) return -FLT_MAX;
        else if constexpr (DT == MX_FLOAT16) return -65504.0f;
        else if constexpr (DT == MX_BFLOAT16) return -3.38953138925153547590470800371487867e38f;  // -0x1.fep127
        else if constexpr (DT == MX_BOOL) return 0;
        else return std::numeric_limits<C>::lowest();
    }
    __device__ __forceinline__ static C highest() {
        if constexpr (DT == MX_FLOAT32) return FLT_MAX;
        else if constexpr (DT == MX_FLOAT16) return 65504.0f;
        else if constexpr (DT == MX_BFLOAT16) return 3.38953138925153547590470800371487867e38f;
        else if constexpr (DT == MX_BOOL) return 1;
        else return std::numeric_limits<C>::max();
    }
};

// Sum state
template <int DT, typename Enable = void> struct SumRed {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    using OutT = S;
    // float for 16/32-bit floats, wrap-around unsigned for integers, OR for bool
    using St = std::conditional_t<Tr::is_float, float,
               std::conditional_t<(sizeof(S) <= 4), uint32_t, uint64_t>>;
    __device__ __forceinline__ static St init() { return St(0); }
    __device__ __forceinline__ static void step(St& s, S x, uint32_t) {
        if constexpr (Tr::is_float) s += Tr::ld(x);
        else if constexpr (DT == MX_BOOL) s |= (St)x;
        else s += (St)x;
    }
    __device__ __forceinline__ static St combine(St a, St b) {
        if constexpr (DT == MX_BOOL) return a | b;
        else return a + b;
    }
    __device__ __forceinline__ static St shfl(St a, int m) { return shfl_x(a, m); }
    __device__ __forceinline__ static OutT out(St s) {
        if constexpr (Tr::is_float) return Tr::st(s);
        else if constexpr (DT == MX_BOOL) return (OutT)(s != 0);
        else return (OutT)s;
    }
};

// (value, first index) state for Max / Min / ArgMax / ArgMin.
template <typename C> struct VI { C v; uint32_t i; };

template <int DT, bool IS_MAX, bool IS_ARG> struct ExtRed {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    using C = typename Tr::C;
    using OutT = std::conditional_t<IS_ARG, int32_t, S>;
    using St = VI<C>;
    __device__ __forceinline__ static bool better(C x, C cur) { return IS_MAX ? (cur < x) : (x < cur); }
    __device__ __forceinline__ static St init() {
        return St{IS_MAX ? Limits<DT>::lowest() : Limits<DT>::highest(), kEmpty};
    }
    __device__ __forceinline__ static void step(St& s, S x, uint32_t idx) {
        C v = Tr::ld(x);
        if (better(v, s.v)) { s.v = v; s.i = idx; }
    }
    __device__ __forceinline__ static St combine(St a, St b) {
        // b wins when strictly better, or equal and earlier (two empties keep a)
        bool take = better(b.v, a.v) || (!better(a.v, b.v) && b.i < a.i);
        return take ? b : a;
    }
    __device__ __forceinline__ static St shfl(St a, int m) {
        St r; r.v = shfl_x(a.v, m); r.i = shfl_x(a.i, m); return r;
    }
    __device__ __forceinline__ static OutT out(St s) {
        if constexpr (IS_ARG) return (int32_t)(s.i == kEmpty ? 0u : s.i);
        else {
            if (s.i == kEmpty) return Tr::st(IS_MAX ? Limits<DT>::lowest() : Limits<DT>::highest());
            return Tr::st(s.v);
        }
    }
};

template <int DT, int OP> struct RedSel;
template <int DT> struct RedSel<DT, MX_RED_SUM> { using R = SumRed<DT>; };
template <int DT> struct RedSel<DT, MX_RED_MAX> { using R = ExtRed<DT, true, false>; };
template <int DT> struct RedSel<DT, MX_RED_MIN> { using R = ExtRed<DT, false, false>; };
template <int DT> struct RedSel<DT, MX_RED_ARGMAX> { using R = ExtRed<DT, true, true>; };
template <int DT> struct RedSel<DT, MX_RED_ARGMIN> { using R = ExtRed<DT, false, true>; };

// ------------------------------------------------------------------ descriptors
struct OffDesc {                       // offset of output g = sum_i (g / sOut_i ...) * sIn_i
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

template <typename S, int VEC> struct alignas(VEC * sizeof(S) >= 16 ? 16 : VEC * sizeof(S)) VecT { S v[VEC]; };

// ------------------------------------------------------------------ kernels
// rows: L lanes per output, reduce stride 1.
template <int DT, int OP, int VEC, int L>
__global__ __launch_bounds__(kBlock) void reduce_rows_kernel(
    typename RedSel<DT, OP>::R::OutT* __restrict__ out, const typename dt_traits<DT>::S* __restrict__ in,
    uint32_t total_out, uint32_t n, OffDesc od) {
    using R = typename RedSel<DT, OP>::R;
    using S = typename dt_traits<DT>::S;
    using V = VecT<S, VEC>;
    const uint64_t tid = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    const uint32_t g = (uint32_t)(tid / L);
    const uint32_t lane = (uint32_t)(tid % L);
    typename R::St st = R::init();
    if (g < total_out) {
        const S* row = in + od.offset(g);
        for (uint32_t e = lane * VEC; e < n; e += L * VEC) {
            V v = *reinterpret_cast<const V*>(row + e);
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st, v.v[k], e + k);
        }
    }
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) st = R::combine(st, R::shfl(st, m));
    if (g < total_out && lane == 0) out[g] = R::out(st);
}

// block: one 256-thread block per (output, chunk); chunk partials go to the workspace.
template <int DT, int OP, int VEC>
__global__ __launch_bounds__(kBlock) void reduce_block_kernel(
    typename RedSel<DT, OP>::R::OutT* __restrict__ out, typename RedSel<DT, OP>::R::St* __restrict__ ws,
    const typename dt_traits<DT>::S* __restrict__ in, uint32_t total_out, uint32_t n,
    uint32_t chunk, uint32_t nchunks, OffDesc od) {
    using R = typename RedSel<DT, OP>::R;
    using S = typename dt_traits<DT>::S;
    using V = VecT<S, VEC>;
    using St = typename R::St;
    constexpr int U = 4;
    const uint32_t g = blockIdx.x;     // outputs on x (up to 2^31), chunks on y (<= 2048)
    const uint32_t c = blockIdx.y;
    const uint32_t beg = c * chunk;
    const uint32_t end = min(n, beg + chunk);
    const S* row = in + od.offset(g);
    St st = R::init();
    uint32_t e = beg + threadIdx.x * VEC;
    for (; e + (U - 1) * kBlock * VEC < end; e += U * kBlock * VEC) {
        V v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = *reinterpret_cast<const V*>(row + e + u * kBlock * VEC);
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st, v[u].v[k], e + u * kBlock * VEC + k);
    }
    for (; e < end; e += kBlock * VEC) {
        V v = *reinterpret_cast<const V*>(row + e);
#pragma unroll
        for (int k = 0; k < VEC; k++) R::step(st, v.v[k], e + k);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) st = R::combine(st, R::shfl(st, m));
    __shared__ St part[kBlock / 64];
    const int wave = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) part[wave] = st;
    __syncthreads();
    if (threadIdx.x == 0) {
        St r = part[0];
#pragma unroll
        for (int w = 1; w < kBlock / 64; w++) r = R::combine(r, part[w]);
        if (nchunks == 1) out[g] = R::out(r);
        else ws[(uint64_t)c * total_out + g] = r;
    }
}

// cols: a thread owns VEC consecutive outputs and walks the reduced axis (chunk c of it).
template <int DT, int OP, int VEC>
__global__ __launch_bounds__(kBlock) void reduce_cols_kernel(
    typename RedSel<DT, OP>::R::OutT* __restrict__ out, typename RedSel<DT, OP>::R::St* __restrict__ ws,
    const typename dt_traits<DT>::S* __restrict__ in, uint32_t total_out, uint32_t n,
    uint32_t rs, uint32_t chunk, uint32_t nchunks, OffDesc od) {
    using R = typename RedSel<DT, OP>::R;
    using S = typename dt_traits<DT>::S;
    using V = VecT<S, VEC>;
    using St = typename R::St;
    constexpr int U = 4;
    const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t g0 = t * VEC;
    if (g0 >= total_out) return;
    const uint32_t c = blockIdx.y;
    const uint32_t beg = c * chunk;
    const uint32_t end = min(n, beg + chunk);
    const S* base = in + od.offset(g0);
    St st[VEC];
#pragma unroll
    for (int k = 0; k < VEC; k++) st[k] = R::init();
    uint32_t i = beg;
    for (; i + U <= end; i += U) {
        V v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = *reinterpret_cast<const V*>(base + (uint64_t)(i + u) * rs);
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int k = 0; k < VEC; k++) R::step(st[k], v[u].v[k], i + u);
    }
    for (; i < end; i++) {
        V v = *reinterpret_cast<const V*>(base + (uint64_t)i * rs);
#pragma unroll
        for (int k = 0; k < VEC; k++) R::step(st[k], v.v[k], i);
    }
#pragma unroll
    for (int k = 0; k < VEC; k++) {
        if (nchunks == 1) out[g0 + k] = R::out(st[k]);
        else ws[(uint64_t)c * total_out + g0 + k] = st[k];
    }
}

// finalize: combine chunk partials in chunk order.
template <int DT, int OP>
__global__ __launch_bounds__(kBlock) void reduce_finalize_kernel(
    typename RedSel<DT, OP>::R::OutT* __restrict__ out, const typename RedSel<DT, OP>::R::St* __restrict__ ws,
    uint32_t total_out, uint32_t nchunks) {
    using R = typename RedSel<DT, OP>::R;
    const uint32_t g = blockIdx.x * kBlock + threadIdx.x;
    if (g >= total_out) return;
    typename R::St r = ws[g];
    for (uint32_t c = 1; c < nchunks; c++) r = R::combine(r, ws[(uint64_t)c * total_out + g]);
    out[g] = R::out(r);
}

// ------------------------------------------------------------------ planning
enum Mode { kRows = 0, kBlockMode = 1, kCols = 2 };

struct Plan {
    Mode mode = kCols;
    int vec = 1;
    int lanes = 1;
    uint32_t nchunks = 1;
    uint32_t chunk = 0;
    uint32_t total_out = 0;
    size_t state_bytes = 0;
    size_t ws_bytes() const { return nchunks > 1 ? (size_t)nchunks * total_out * state_bytes : 0; }
};

template <int DT, int OP>
size_t state_size() { return sizeof(typename RedSel<DT, OP>::R::St); }

struct Desc {
    int cd;
    uint32_t shape[MX_MAX_DIMS], so[MX_MAX_DIMS], si[MX_MAX_DIMS];
    uint32_t rs, n;
};

// The chunking depends only on the descriptor (never on pointer alignment), so the
// workspace size reported ahead of time always covers the launch.
Plan make_plan(const Desc& d, size_t elem, size_t stbytes, uintptr_t in_ptr) {
    Plan p;
    uint64_t tot = 1;
    for (int i = 0; i < d.cd; i++) tot *= d.shape[i];
    p.total_out = (uint32_t)tot;
    p.state_bytes = stbytes;
    const int VEC = (int)(16 / elem);
    const bool aligned = in_ptr % 16 == 0;
    if (d.rs == 1 && d.n > 1) {
        bool v_ok = VEC > 1 && d.n % VEC == 0;
        for (int i = 0; v_ok && i < d.cd; i++) if (d.si[i] % VEC) v_ok = false;
        const uint32_t nominal = v_ok ? (uint32_t)VEC : 1u;
        p.vec = (v_ok && aligned) ? VEC : 1;
        const uint32_t nv = (d.n + nominal - 1) / nominal;
        if (nv > 1024) {
            p.mode = kBlockMode;
            const uint32_t per_block = 2048;      // vectors per block (8 per thread)
            uint64_t want = (2048 + tot - 1) / tot;
            uint64_t maxc = (nv + per_block - 1) / per_block;
            uint64_t nc = want < maxc ? want : maxc;
            if (nc < 1) nc = 1;
            uint32_t chunk_v = (uint32_t)((nv + nc - 1) / nc);
            p.chunk = chunk_v * nominal;
            p.nchunks = (d.n + p.chunk - 1) / p.chunk;
        } else {
            p.mode = kRows;
            p.lanes = nv <= 2 ? 1 : nv <= 16 ? 4 : nv <= 64 ? 16 : 64;
        }
        return p;
    }
    // column / general
    const int last = d.cd - 1;
    bool v_ok = VEC > 1 && d.so[last] == 1 && d.si[last] == 1 && d.shape[last] % VEC == 0 &&
                d.rs % VEC == 0;
    for (int i = 0; v_ok && i < last; i++) if (d.si[i] % VEC || d.so[i] % VEC) v_ok = false;
    p.mode = kCols;
    p.vec = (v_ok && aligned) ? VEC : 1;
    const uint64_t threads = tot / (v_ok ? VEC : 1);
    p.nchunks = 1;
    if (d.n >= 64 && threads < 131072) {
        uint64_t want = (131072 + threads - 1) / threads;
        uint64_t maxc = d.n / 16;
        if (maxc > 4096) maxc = 4096;          // grid.y stays far below its 65535 limit
        uint64_t nc = want < maxc ? want : maxc;
        if (nc > 1) {
            p.chunk = (uint32_t)((d.n + nc - 1) / nc);
            p.nchunks = (d.n + p.chunk - 1) / p.chunk;
        }
    }
    if (p.nchunks == 1) p.chunk = d.n;
    return p;
}

template <int DT, int OP>
int run(const Desc& d, void* outp, const void* inp, void* ws, size_t ws_bytes, hipStream_t st) {
    using R = typename RedSel<DT, OP>::R;
    using S = typename dt_traits<DT>::S;
    using OutT = typename R::OutT;
    using StT = typename R::St;
    constexpr int VEC = 16 / sizeof(S);
    Plan p = make_plan(d, sizeof(S), sizeof(StT), (uintptr_t)inp);
    if (p.total_out == 0) return MX_OK;
    if (p.ws_bytes() > 0 && (ws == nullptr || ws_bytes < p.ws_bytes()))
        return fail(MX_ERR_WORKSPACE, "mx_launch_reduce: workspace of " + std::to_string(p.ws_bytes()) +
                                          " bytes required, " + std::to_string(ws_bytes) + " given");
    OffDesc od{};
    od.n = d.cd;
    for (int i = 0; i < d.cd; i++) { od.so[i] = FastDiv(d.so[i]); od.si[i] = d.si[i]; }
    OutT* out = (OutT*)outp;
    const S* in = (const S*)inp;
    StT* wsp = (StT*)ws;
    if (p.mode == kRows) {
        uint64_t threads = (uint64_t)p.total_out * p.lanes;
        dim3 grid((uint32_t)((threads + kBlock - 1) / kBlock));
#define MX_ROWS(V_, L_) hipLaunchKernelGGL((reduce_rows_kernel<DT, OP, V_, L_>), grid, dim3(kBlock), 0, st, out, in, p.total_out, d.n, od)
        if (p.vec == VEC && VEC > 1) {
            switch (p.lanes) { case 1: MX_ROWS(VEC, 1); break; case 4: MX_ROWS(VEC, 4); break;
                               case 16: MX_ROWS(VEC, 16); break; default: MX_ROWS(VEC, 64); break; }
        } else {
            switch (p.lanes) { case 1: MX_ROWS(1, 1); break; case 4: MX_ROWS(1, 4); break;
                               case 16: MX_ROWS(1, 16); break; default: MX_ROWS(1, 64); break; }
        }
#undef MX_ROWS
    } else if (p.mode == kBlockMode) {
        dim3 grid(p.total_out, p.nchunks);
        if (p.vec == VEC && VEC > 1)
            hipLaunchKernelGGL((reduce_block_kernel<DT, OP, VEC>), grid, dim3(kBlock), 0, st, out, wsp, in, p.total_out, d.n, p.chunk, p.nchunks, od);
        else
            hipLaunchKernelGGL((reduce_block_kernel<DT, OP, 1>), grid, dim3(kBlock), 0, st, out, wsp, in, p.total_out, d.n, p.chunk, p.nchunks, od);
    } else {
        uint32_t threads = p.total_out / p.vec;
        dim3 grid((threads + kBlock - 1) / kBlock, p.nchunks);
        if (p.vec == VEC && VEC > 1)
            hipLaunchKernelGGL((reduce_cols_kernel<DT, OP, VEC>), grid, dim3(kBlock), 0, st, out, wsp, in, p.total_out, d.n, d.rs, p.chunk, p.nchunks, od);
        else
            hipLaunchKernelGGL((reduce_cols_kernel<DT, OP, 1>), grid, dim3(kBlock), 0, st, out, wsp, in, p.total_out, d.n, d.rs, p.chunk, p.nchunks, od);
    }
    MX_HIP(hipGetLastError());
    if (p.nchunks > 1) {
        dim3 grid((p.total_out + kBlock - 1) / kBlock);
        hipLaunchKernelGGL((reduce_finalize_kernel<DT, OP>), grid, dim3(kBlock), 0, st, out, wsp, p.total_out, p.nchunks);
        MX_HIP(hipGetLastError());
    }
    return MX_OK;
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

using namespace mx;

extern "C" int mx_reduce_workspace_bytes(int op, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                                         int cdims, const uint32_t* shape, const uint32_t* sOut,
                                         const uint32_t* sIn, size_t* bytes) {
    if (!bytes) return fail(MX_ERR_INVALID_ARG, "mx_reduce_workspace_bytes: null out pointer");
    Desc d;
    int rc = check_desc("mx_reduce_workspace_bytes", op, cdims, shape, sOut, sIn, reduce_stride, n_reduce, &d);
    if (rc != MX_OK) return rc;
    size_t st = 0, el = 0;
    bool ok = dispatch_dtype(dtype, [&](auto dt) {
        constexpr int DT = decltype(dt)::value;
        el = sizeof(typename dt_traits<DT>::S);
        dispatch_op(op, [&](auto o) { st = state_size<DT, decltype(o)::value>(); });
    });
    if (!ok) return fail(MX_ERR_UNSUPPORTED, "mx_reduce_workspace_bytes: no kernel for dtype " + std::to_string(dtype));
    // Alignment only changes the vector width, never the chunking of the column plan; the
    // row plan's chunking depends on it, so size for the worst case (aligned input).
    Plan p = make_plan(d, el, st, 0);
    *bytes = p.ws_bytes();
    return MX_OK;
}

extern "C" int mx_launch_reduce(int op, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                                int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                                void* out, const void* in, void* workspace, size_t workspace_bytes,
                                void* stream) {
    Desc d;
    int rc = check_desc("mx_launch_reduce", op, cdims, shape, sOut, sIn, reduce_stride, n_reduce, &d);
    if (rc != MX_OK) return rc;
    uint64_t tot = 1;
    for (int i = 0; i < d.cd; i++) tot *= d.shape[i];
    if (tot == 0) return MX_OK;
    if (!out || (!in && n_reduce > 0)) return fail(MX_ERR_INVALID_ARG, "mx_launch_reduce: null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    rc = MX_OK;
    bool ok = dispatch_dtype(dtype, [&](auto dt) {
        constexpr int DT = decltype(dt)::value;
        dispatch_op(op, [&](auto o) { rc = run<DT, decltype(o)::value>(d, out, in, workspace, workspace_bytes, st); });
    });
    if (!ok) return fail(MX_ERR_UNSUPPORTED, "mx_launch_reduce: no kernel for dtype " + std::to_string(dtype));
    return rc;
}
