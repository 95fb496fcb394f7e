// reduce_group_impl.hpp -- the group kernels of mx_launch_reduce_group and their launcher,
// run_reduce_group<DT>, instantiated once per float dtype (reduce_group_f32.hip, _f16, _bf16) so
// the three compile in parallel.  A member runs the same plan body as its single-op kernel
// (reduce_plans.hpp); blockIdx.z selects the member and a uniform switch its op.
#pragma once
#include "reduce_plans.hpp"

namespace mx {
namespace {

// ------------------------------------------------------------------ group kernels
// The member's pointers, typed for its op.
#define MX_GROUP_MEMBER(OP_)                                                                    \
    constexpr int OP = decltype(OP_)::value;                                                    \
    OutOf<DT, OP>* out = static_cast<OutOf<DT, OP>*>(gp.out[k]);                                \
    StOf<DT, OP>* part = static_cast<StOf<DT, OP>*>(gp.part[k]);                                \
    const ElemOf<DT>* in = static_cast<const ElemOf<DT>*>(gp.in[k]);                            \
    (void)out; (void)part; (void)in

template <int DT, int VEC, int L, int U>
__global__ __launch_bounds__(256) void reduce_rows_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t n,
                                                                uint32_t rounds, OffDesc od) {
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        rows_body<DT, OP, VEC, L, U>(out, in, total_out, n, rounds, od, blockIdx.x, gridDim.x);
    });
}

template <int DT, int VEC, int NV>
__global__ __launch_bounds__(256) void reduce_lane_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t nv,
                                                                OffDesc od) {
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        lane_body<DT, OP, VEC, NV>(out, in, total_out, nv, od, blockIdx.x);
    });
}

template <int DT, int VEC>
__global__ __launch_bounds__(256) void reduce_lane_packed_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t nv) {
    __shared__ VecT<ElemOf<DT>, VEC> sh[1024];
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        lane_packed_body<DT, OP, VEC>(out, in, total_out, nv, blockIdx.x, sh);
    });
}

template <int DT, int VEC, int WAVES, int U>
__global__ __launch_bounds__(64 * WAVES) void reduce_block_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t n,
                                                                        uint32_t chunk, uint32_t nsplit, OffDesc od) {
    __shared__ __align__(16) char smem[WAVES * kMaxState<DT>];
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        block_body<DT, OP, VEC, WAVES, U>(out, part, in, total_out, n, chunk, nsplit, od, blockIdx.x, blockIdx.y, smem);
    });
}

template <int DT, int VEC, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void reduce_cols_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t n,
                                                                       uint32_t rs, uint32_t chunk, uint32_t nsplit,
                                                                       OffDesc od) {
    __shared__ __align__(16) char smem[(WAVES > 1 ? (WAVES - 1) * 64 * VEC : 1) * kMaxState<DT>];
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        cols_body<DT, OP, VEC, WAVES>(out, part, in, total_out, n, rs, chunk, nsplit, od, blockIdx.x, blockIdx.y, smem);
    });
}

// VST_OK: outputs 16-byte aligned; a member stores VEC outputs at once when they make 16 bytes.
template <int DT, int VEC, int NMAX, int WAVES, bool VST_OK>
__global__ __launch_bounds__(64 * WAVES) void reduce_short_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t n,
                                                                        uint32_t rs, OffDesc od) {
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        constexpr bool kVst = VST_OK && sizeof(OutOf<DT, OP>) * VEC == 16;
        short_body<DT, OP, VEC, NMAX, WAVES, kVst>(out, in, total_out, n, rs, od, blockIdx.x);
    });
}

template <int DT>
__global__ __launch_bounds__(256) void reduce_finalize_group_kernel(GroupPtrs gp, uint32_t total_out, uint32_t nsplit) {
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        finalize_body<DT, OP>(out, part, total_out, nsplit, blockIdx.x);
    });
}

template <int DT>
__global__ __launch_bounds__(256) void reduce_finalize_wide_group_kernel(GroupPtrs gp, uint32_t total_out,
                                                                         uint32_t nsplit) {
    __shared__ __align__(16) char smem[4 * kMaxState<DT>];
    const int k = blockIdx.z;
    op_switch(gp.op[k], [&](auto o) {
        MX_GROUP_MEMBER(o);
        finalize_wide_body<DT, OP>(out, part, total_out, nsplit, blockIdx.x, smem);
    });
}
#undef MX_GROUP_MEMBER

}  // namespace

// A group of n reductions of one dtype over one descriptor: one launch of the plan's group kernel
// (blockIdx.z = member) and, when the plan splits the axis, one combine launch.  The members share
// the plan: vector loads only when every input is 16-byte aligned, vector stores (short plan) only
// when every output is.  Each member's results are those of its own mx_launch_reduce.
template <int DT>
int run_reduce_group(const Desc& d, int n, const int* ops, void* const* outs, const void* const* ins, void* const* ws,
              const size_t* ws_bytes, hipStream_t st) {
    using S = ElemOf<DT>;
    constexpr int VEC = 16 / sizeof(S);
    uintptr_t in_or = 0;
    bool out_aligned = true;
    for (int k = 0; k < n; k++) {
        in_or |= (uintptr_t)ins[k];
        out_aligned = out_aligned && (uintptr_t)outs[k] % 16 == 0;
    }
    const Plan p = make_plan(d, sizeof(S), 0, in_or);
    if (p.total_out == 0) return MX_OK;
    GroupPtrs gp{};
    for (int k = 0; k < n; k++) {
        size_t stb = 0;
        dispatch_op(ops[k], [&](auto o) { stb = sizeof(StOf<DT, decltype(o)::value>); });
        const size_t need = p.nsplit > 1 ? (size_t)p.nsplit * p.total_out * stb : 0;
        if (need > 0 && (!ws || !ws_bytes || !ws[k] || ws_bytes[k] < need))
            return fail(MX_ERR_WORKSPACE, "mx_launch_reduce_group: member " + std::to_string(k) + " needs a workspace of " +
                                              std::to_string(need) + " bytes (mx_reduce_workspace_bytes)");
        gp.op[k] = ops[k];
        gp.in[k] = ins[k];
        gp.out[k] = outs[k];
        gp.part[k] = need ? ws[k] : nullptr;
    }
    OffDesc od{};
    od.n = d.cd;
    for (int i = 0; i < d.cd; i++) { od.so[i] = FastDiv(d.so[i]); od.si[i] = d.si[i]; }
    const bool vec = p.vec == VEC && VEC > 1;
    const uint32_t nz = (uint32_t)n;
    if (p.mode == kLane) {
        const dim3 grid(p.blocks, 1, nz);
        if (p.packed) hipLaunchKernelGGL((reduce_lane_packed_group_kernel<DT, VEC>), grid, dim3(256), 0, st, gp, p.total_out, p.nv);
        else if (vec) hipLaunchKernelGGL((reduce_lane_group_kernel<DT, VEC, 4>), grid, dim3(256), 0, st, gp, p.total_out, p.nv, od);
        else hipLaunchKernelGGL((reduce_lane_group_kernel<DT, 1, 4>), grid, dim3(256), 0, st, gp, p.total_out, p.nv, od);
    } else if (p.mode == kShort) {
        const uint32_t gx = (uint32_t)((p.total_out + 64ull * p.waves * p.vec - 1) / (64ull * p.waves * p.vec));
        const dim3 grid(gx, 1, nz);
#define MX_SHORT(V_, W_, VST_) hipLaunchKernelGGL((reduce_short_group_kernel<DT, V_, 8, W_, VST_>), grid, dim3(64 * W_), 0, \
                                                  st, gp, p.total_out, d.n, d.rs, od)
        if (vec && out_aligned) { if (p.waves == 1) MX_SHORT(VEC, 1, true); else MX_SHORT(VEC, 4, true); }
        else if (vec) { if (p.waves == 1) MX_SHORT(VEC, 1, false); else MX_SHORT(VEC, 4, false); }
        else { if (p.waves == 1) MX_SHORT(1, 1, false); else MX_SHORT(1, 4, false); }
#undef MX_SHORT
    } else if (p.mode == kRows) {
        const dim3 grid(p.blocks, 1, nz);
#define MX_ROWS(V_, L_, U_) hipLaunchKernelGGL((reduce_rows_group_kernel<DT, V_, L_, U_>), grid, dim3(256), 0, st, gp, \
                                               p.total_out, d.n, p.rounds, od)
        if (vec) {
            switch (p.lanes) { case 1: MX_ROWS(VEC, 1, 4); break; case 4: MX_ROWS(VEC, 4, 4); break;
                               case 16: MX_ROWS(VEC, 16, 4); break; default: MX_ROWS(VEC, 64, 1); break; }
        } else {
            switch (p.lanes) { case 1: MX_ROWS(1, 1, 4); break; case 4: MX_ROWS(1, 4, 4); break;
                               case 16: MX_ROWS(1, 16, 4); break; default: MX_ROWS(1, 64, 1); break; }
        }
#undef MX_ROWS
    } else if (p.mode == kBlockMode) {
        const dim3 grid(p.total_out, p.nsplit, nz);
#define MX_BLOCK(V_, W_, U_) hipLaunchKernelGGL((reduce_block_group_kernel<DT, V_, W_, U_>), grid, dim3(64 * W_), 0, st, \
                                                gp, p.total_out, d.n, p.chunk, p.nsplit, od)
        if (vec) { if (p.waves == 16) MX_BLOCK(VEC, 16, 4); else MX_BLOCK(VEC, 4, 8); }
        else { if (p.waves == 16) MX_BLOCK(1, 16, 4); else MX_BLOCK(1, 4, 8); }
#undef MX_BLOCK
    } else {
        const uint32_t gx = (uint32_t)((p.total_out + 64ull * p.vec - 1) / (64ull * p.vec));
        const dim3 grid(gx, p.nsplit, nz);
        if (vec) hipLaunchKernelGGL((reduce_cols_group_kernel<DT, VEC, 4>), grid, dim3(256), 0, st, gp, p.total_out, d.n,
                                    d.rs, p.chunk, p.nsplit, od);
        else hipLaunchKernelGGL((reduce_cols_group_kernel<DT, 1, 4>), grid, dim3(256), 0, st, gp, p.total_out, d.n, d.rs,
                                p.chunk, p.nsplit, od);
    }
    MX_HIP(hipGetLastError());
    if (p.nsplit > 32 && p.total_out <= 65535u * 16) {
        hipLaunchKernelGGL((reduce_finalize_wide_group_kernel<DT>), dim3(p.total_out, 1, nz), dim3(256), 0, st, gp,
                           p.total_out, p.nsplit);
        MX_HIP(hipGetLastError());
    } else if (p.nsplit > 1) {
        hipLaunchKernelGGL((reduce_finalize_group_kernel<DT>), dim3((p.total_out + 255) / 256, 1, nz), dim3(256), 0, st,
                           gp, p.total_out, p.nsplit);
        MX_HIP(hipGetLastError());
    }
    return MX_OK;
}

}  // namespace mx
