// reduce.hip -- Sum / Max / Min / ArgMax / ArgMin over one axis: one launch per reduction (plus
// one combine launch for a split axis).  The plans, their semantics and their choice are in
// reduce_plans.hpp.
#include "reduce_plans.hpp"

#include <mutex>

namespace mx {
namespace {

template <int DT, int OP, int VEC, int L, int U>
__global__ __launch_bounds__(256) void reduce_rows_kernel(OutOf<DT, OP>* __restrict__ out,
                                                          const ElemOf<DT>* __restrict__ in, uint32_t total_out,
                                                          uint32_t n, uint32_t rounds, OffDesc od) {
    rows_body<DT, OP, VEC, L, U>(out, in, total_out, n, rounds, od, blockIdx.x, gridDim.x);
}

template <int DT, int OP, int VEC, int NV>
__global__ __launch_bounds__(256) void reduce_lane_kernel(OutOf<DT, OP>* __restrict__ out,
                                                          const ElemOf<DT>* __restrict__ in, uint32_t total_out,
                                                          uint32_t nv, OffDesc od) {
    lane_body<DT, OP, VEC, NV>(out, in, total_out, nv, od, blockIdx.x);
}

template <int DT, int OP, int VEC>
__global__ __launch_bounds__(256) void reduce_lane_packed_kernel(OutOf<DT, OP>* __restrict__ out,
                                                                 const ElemOf<DT>* __restrict__ in, uint32_t total_out,
                                                                 uint32_t nv) {
    __shared__ VecT<ElemOf<DT>, VEC> sh[1024];
    lane_packed_body<DT, OP, VEC>(out, in, total_out, nv, blockIdx.x, sh);
}

template <int DT, int OP, int VEC, int WAVES, int U>
__global__ __launch_bounds__(64 * WAVES) void reduce_block_kernel(OutOf<DT, OP>* __restrict__ out,
                                                                  StOf<DT, OP>* __restrict__ part,
                                                                  const ElemOf<DT>* __restrict__ in, uint32_t total_out,
                                                                  uint32_t n, uint32_t chunk, uint32_t nsplit,
                                                                  OffDesc od) {
    __shared__ StOf<DT, OP> wpart[WAVES];
    block_body<DT, OP, VEC, WAVES, U>(out, part, in, total_out, n, chunk, nsplit, od, blockIdx.x, blockIdx.y, wpart);
}

template <int DT, int OP, int VEC, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void reduce_cols_kernel(OutOf<DT, OP>* __restrict__ out,
                                                                 StOf<DT, OP>* __restrict__ part,
                                                                 const ElemOf<DT>* __restrict__ in, uint32_t total_out,
                                                                 uint32_t n, uint32_t rs, uint32_t chunk, uint32_t nsplit,
                                                                 OffDesc od) {
    __shared__ StOf<DT, OP> sh[WAVES > 1 ? (WAVES - 1) * 64 * VEC : 1];
    cols_body<DT, OP, VEC, WAVES>(out, part, in, total_out, n, rs, chunk, nsplit, od, blockIdx.x, blockIdx.y, sh);
}

template <int DT, int OP, int VEC, int NMAX, int WAVES, bool VST>
__global__ __launch_bounds__(64 * WAVES) void reduce_short_kernel(OutOf<DT, OP>* __restrict__ out,
                                                                  const ElemOf<DT>* __restrict__ in, uint32_t total_out,
                                                                  uint32_t n, uint32_t rs, OffDesc od) {
    short_body<DT, OP, VEC, NMAX, WAVES, VST>(out, in, total_out, n, rs, od, blockIdx.x);
}

template <int DT, int OP>
__global__ __launch_bounds__(256) void reduce_finalize_kernel(OutOf<DT, OP>* __restrict__ out,
                                                              const StOf<DT, OP>* __restrict__ part, uint32_t total_out,
                                                              uint32_t nsplit) {
    finalize_body<DT, OP>(out, part, total_out, nsplit, blockIdx.x);
}

template <int DT, int OP>
__global__ __launch_bounds__(256) void reduce_finalize_wide_kernel(OutOf<DT, OP>* __restrict__ out,
                                                                   const StOf<DT, OP>* __restrict__ part,
                                                                   uint32_t total_out, uint32_t nsplit) {
    __shared__ StOf<DT, OP> w[4];
    finalize_wide_body<DT, OP>(out, part, total_out, nsplit, blockIdx.x, w);
}

template <int DT, int OP>
size_t state_size() { return sizeof(typename RedSel<DT, OP>::R::St); }

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
    StT* part = (StT*)ws;
    const bool vec = p.vec == VEC && VEC > 1;
    if (p.mode == kLane) {
        dim3 grid(p.blocks);
        if (p.packed) hipLaunchKernelGGL((reduce_lane_packed_kernel<DT, OP, VEC>), grid, dim3(256), 0, st, out, in, p.total_out, p.nv);
        else if (vec) hipLaunchKernelGGL((reduce_lane_kernel<DT, OP, VEC, 4>), grid, dim3(256), 0, st, out, in, p.total_out, p.nv, od);
        else hipLaunchKernelGGL((reduce_lane_kernel<DT, OP, 1, 4>), grid, dim3(256), 0, st, out, in, p.total_out, p.nv, od);
    } else if (p.mode == kShort) {
        const uint32_t gx = (uint32_t)((p.total_out + 64ull * p.waves * p.vec - 1) / (64ull * p.waves * p.vec));
#define MX_SHORT(V_, W_, VST_) hipLaunchKernelGGL((reduce_short_kernel<DT, OP, V_, 8, W_, VST_>), dim3(gx), dim3(64 * W_), 0, st, \
                                                  out, in, p.total_out, d.n, d.rs, od)
        constexpr bool kVst = sizeof(OutT) * VEC == 16;   // VEC outputs fill one 128-bit store
        bool done = false;
        if constexpr (kVst) {
            if (vec && (uintptr_t)outp % 16 == 0) {
                if (p.waves == 1) MX_SHORT(VEC, 1, true); else MX_SHORT(VEC, 4, true);
                done = true;
            }
        }
        if (!done) {
            if (vec) { if (p.waves == 1) MX_SHORT(VEC, 1, false); else MX_SHORT(VEC, 4, false); }
            else { if (p.waves == 1) MX_SHORT(1, 1, false); else MX_SHORT(1, 4, false); }
        }
#undef MX_SHORT
    } else if (p.mode == kRows) {
        dim3 grid(p.blocks);
#define MX_ROWS(V_, L_, U_) hipLaunchKernelGGL((reduce_rows_kernel<DT, OP, V_, L_, U_>), grid, dim3(256), 0, st, \
                                               out, in, p.total_out, d.n, p.rounds, od)
        if (vec) {
            switch (p.lanes) { case 1: MX_ROWS(VEC, 1, 4); break; case 4: MX_ROWS(VEC, 4, 4); break;
                               case 16: MX_ROWS(VEC, 16, 4); break; default: MX_ROWS(VEC, 64, 1); break; }
        } else {
            switch (p.lanes) { case 1: MX_ROWS(1, 1, 4); break; case 4: MX_ROWS(1, 4, 4); break;
                               case 16: MX_ROWS(1, 16, 4); break; default: MX_ROWS(1, 64, 1); break; }
        }
#undef MX_ROWS
    } else if (p.mode == kBlockMode) {
        dim3 grid(p.total_out, p.nsplit);
#define MX_BLOCK(V_, W_, U_) hipLaunchKernelGGL((reduce_block_kernel<DT, OP, V_, W_, U_>), grid, dim3(64 * W_), 0, st, \
                                                out, part, in, p.total_out, d.n, p.chunk, p.nsplit, od)
        if (vec) {
            if (p.waves == 16) MX_BLOCK(VEC, 16, 4); else MX_BLOCK(VEC, 4, 8);
        } else {
            if (p.waves == 16) MX_BLOCK(1, 16, 4); else MX_BLOCK(1, 4, 8);
        }
#undef MX_BLOCK
    } else {
        // the x extent is in units of 64 lanes x the vector width actually used
        const uint32_t gx = (uint32_t)((p.total_out + 64ull * p.vec - 1) / (64ull * p.vec));
        dim3 grid(gx, p.nsplit);
#define MX_COLS(V_, W_) hipLaunchKernelGGL((reduce_cols_kernel<DT, OP, V_, W_>), grid, dim3(64 * W_), 0, st, \
                                           out, part, in, p.total_out, d.n, d.rs, p.chunk, p.nsplit, od)
        if (vec) MX_COLS(VEC, 4);
        else MX_COLS(1, 4);
#undef MX_COLS
    }
    MX_HIP(hipGetLastError());
    if (p.nsplit > 32 && p.total_out <= 65535u * 16) {
        hipLaunchKernelGGL((reduce_finalize_wide_kernel<DT, OP>), dim3(p.total_out), dim3(256), 0, st, out, part,
                           p.total_out, p.nsplit);
        MX_HIP(hipGetLastError());
    } else if (p.nsplit > 1) {
        dim3 grid((p.total_out + 255) / 256);
        hipLaunchKernelGGL((reduce_finalize_kernel<DT, OP>), grid, dim3(256), 0, st, out, part, p.total_out, p.nsplit);
        MX_HIP(hipGetLastError());
    }
    return MX_OK;
}

}  // namespace
}  // namespace mx


using namespace mx;

// ------------------------------------------------------------------ the allocation-free form
// mx_launch_reduce_noalloc takes its split partials from `scratch`, a fixed device array instead
// of a caller workspace.  Host code never passes `scratch` itself (in host code the name is a
// host-side stand-in, not a device address): mx_hip_init looks up each device's own address of
// the array once, with that device current, and the entry point passes that address.  The
// partials are written by the first launch before the combine launch reads them, so nothing in
// the array has to start at zero.
namespace mx {
constexpr size_t kNoallocScratchBytes = (size_t)4 << 20;
constexpr int kMaxDevices = 64;
}  // namespace mx

static __device__ __align__(256) unsigned char scratch[mx::kNoallocScratchBytes];

namespace mx {
namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// Called by mx_hip_init with `device` current.
int reduce_noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices)
        return fail(MX_ERR_UNSUPPORTED, "mx_hip_init: device " + std::to_string(device) + " beyond the " +
                                            std::to_string(kMaxDevices) + " this library tracks");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return MX_OK;
    void* ptr = nullptr;
    MX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail(MX_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[device] = ptr;
    return MX_OK;
}

}  // namespace mx

extern "C" int mx_launch_reduce_noalloc(int op, int dtype, uint32_t reduce_stride, uint32_t n_reduce, int cdims,
                                        const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn, void* out,
                                        const void* in, void* stream) {
    size_t need = 0;
    int rc = mx_reduce_workspace_bytes(op, dtype, reduce_stride, n_reduce, cdims, shape, sOut, sIn, &need);
    if (rc != MX_OK) return rc;
    if (need > kNoallocScratchBytes)
        return fail(MX_ERR_WORKSPACE, "mx_launch_reduce_noalloc: this reduction needs " + std::to_string(need) +
                                          " bytes of split partials, above the fixed " +
                                          std::to_string(kNoallocScratchBytes) +
                                          " (use mx_launch_reduce with a workspace)");
    void* ws = nullptr;
    if (need > 0) {
        // the array of the GPU the launch runs on: the stream's device
        hipStream_t st;
        if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
        hipDevice_t dev = -1;
        MX_HIP(hipStreamGetDevice(st, &dev));
        {
            std::lock_guard<std::mutex> lk(g_scratch_mu);
            if (dev >= 0 && dev < kMaxDevices) ws = g_scratch_ptr[dev];
        }
        if (!ws)
            return fail(MX_ERR_NOT_INITIALIZED, "mx_launch_reduce_noalloc: device " + std::to_string(dev) +
                                                    " was not set up by mx_hip_init");
    }
    return mx_launch_reduce(op, dtype, reduce_stride, n_reduce, cdims, shape, sOut, sIn, out, in, ws,
                            ws ? kNoallocScratchBytes : 0, stream);
}

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
