// bcast.hip -- broadcast binary kernels: Add / Sub / Mul / Divide / Max / Min / Equal.
//
// Semantics per element follow the reference CPU backends (Matrix.mm:7411-7707,
// Matrix.mm:13378-13478, Matrix.mm:14668-14783, Matrix.mm:14469-14540):
//   - 16-bit floats compute in float and round once (nearest-even) on store;
//   - integers wrap; integer division truncates, a zero divisor gives 0 and MIN / -1 gives
//     MIN (arm64 sdiv / udiv, the reference's platform);
//   - Max is (a < b) ? b : a and Min is (b < a) ? b : a, selecting the operand's own bits
//     (std::max / std::min), so NaN and signed-zero ties resolve as on the CPU;
//   - Equal writes 1 / 0 in the operands' dtype;
//   - complex64 (Add / Sub / Mul / Divide only) follows complex.h:28-52.
//
// Layout: the iteration space is the collapsed CollapsedDims_3 of collapse_dims
// (Mods/Utils.mm:169-202).  When the innermost collapsed axis is unit-stride in the output
// and unit- or zero-stride in each operand, one thread moves 16 bytes per operand with
// 128-bit loads and stores; otherwise a scalar kernel gathers with the full strides.
#include "elementwise.hpp"

namespace mx {
namespace {

constexpr int kMaxOuter = MX_MAX_DIMS - 1;

struct OuterDesc {                  // outer (non-innermost) collapsed axes
    int n;                          // number of outer axes
    FastDiv shape[kMaxOuter];
    uint32_t sA[kMaxOuter], sB[kMaxOuter], sR[kMaxOuter];
};

struct FullDesc {                   // all collapsed axes
    int n;
    FastDiv shape[MX_MAX_DIMS];
    uint32_t sA[MX_MAX_DIMS], sB[MX_MAX_DIMS], sR[MX_MAX_DIMS];
};

template <typename S, int VEC>
struct alignas(16) Vec { S v[VEC]; };

constexpr int kBlock = 256;
// One 16-byte vector per operand per thread: at the workload sizes (16-64 MiB) more vectors per
// thread only lengthen the tail of the launch (measured: 7.0 us for 32 MiB at one vector a
// thread, 7.4-7.7 us at two to four).
constexpr int kUnroll = 1;

// One thread = kUnroll slots of VEC consecutive outputs along the innermost axis.
template <int DT, int OP, int VEC, bool AV, bool BV>
__global__ __launch_bounds__(kBlock) void bcast_vec_kernel(
    typename dt_traits<DT>::S* __restrict__ R, const typename dt_traits<DT>::S* __restrict__ A,
    const typename dt_traits<DT>::S* __restrict__ B, uint32_t nvec, FastDiv inner_vecs,
    OuterDesc od, int nt) {
    using S = typename dt_traits<DT>::S;
    using V = Vec<S, VEC>;
    const uint32_t base = blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    V va[kUnroll], vb[kUnroll];
    uint64_t offR[kUnroll];
    bool live[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        const uint32_t v = base + u * kBlock;
        live[u] = v < nvec;
        if (!live[u]) continue;
        uint32_t row = inner_vecs.div(v);
        uint32_t col = (v - row * inner_vecs.d) * VEC;
        uint64_t oa = 0, ob = 0, orr = 0;
        for (int d = od.n - 1; d >= 0; --d) {
            uint32_t q = od.shape[d].div(row);
            uint32_t idx = row - q * od.shape[d].d;
            row = q;
            oa += (uint64_t)idx * od.sA[d];
            ob += (uint64_t)idx * od.sB[d];
            orr += (uint64_t)idx * od.sR[d];
        }
        offR[u] = orr + col;
        if constexpr (AV) {
            const V* p = reinterpret_cast<const V*>(A + oa + col);
            va[u] = (nt & 1) ? ld_stream(p) : *p;
        }
        else { S s = A[oa];
#pragma unroll
            for (int i = 0; i < VEC; i++) va[u].v[i] = s; }
        if constexpr (BV) {
            const V* p = reinterpret_cast<const V*>(B + ob + col);
            vb[u] = (nt & 2) ? ld_stream(p) : *p;
        }
        else { S s = B[ob];
#pragma unroll
            for (int i = 0; i < VEC; i++) vb[u].v[i] = s; }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
        if (!live[u]) continue;
        V r;
#pragma unroll
        for (int i = 0; i < VEC; i++) r.v[i] = BinOp<DT, OP>::apply(va[u].v[i], vb[u].v[i]);
        *reinterpret_cast<V*>(R + offR[u]) = r;
    }
}

// Scalar gather: one output element per thread, any strides.
template <int DT, int OP>
__global__ __launch_bounds__(kBlock) void bcast_scalar_kernel(
    typename dt_traits<DT>::S* __restrict__ R, const typename dt_traits<DT>::S* __restrict__ A,
    const typename dt_traits<DT>::S* __restrict__ B, uint32_t total, FullDesc fd) {
    uint32_t g = blockIdx.x * kBlock + threadIdx.x;
    if (g >= total) return;
    uint32_t rem = g;
    uint64_t oa = 0, ob = 0, orr = 0;
    for (int d = fd.n - 1; d >= 0; --d) {
        uint32_t q = fd.shape[d].div(rem);
        uint32_t idx = rem - q * fd.shape[d].d;
        rem = q;
        oa += (uint64_t)idx * fd.sA[d];
        ob += (uint64_t)idx * fd.sB[d];
        orr += (uint64_t)idx * fd.sR[d];
    }
    R[orr] = BinOp<DT, OP>::apply(A[oa], B[ob]);
}

// ------------------------------------------------------------------ gradient of Max / Min
// The vjp of Max / Min (primitives.cpp:2604-2608) sends g to b where b equals the result and to a
// elsewhere: mask_b = equal(b, max(a, b)), grad_a = g * (1 - mask_b), grad_b = g * mask_b (min for
// Min).  One element of either, with the very operations those four broadcast launches apply
// (compare in float, select the operand's own bits, 1 / 0 and 1 - mask in the dtype, the
// product rounded once), so the result is the same bit for bit.
template <int DT>
__device__ __forceinline__ typename dt_traits<DT>::S max_grad_elem(typename dt_traits<DT>::S a,
                                                                    typename dt_traits<DT>::S b,
                                                                    typename dt_traits<DT>::S g, int op, int side) {
    using Tr = dt_traits<DT>;
    using S = typename Tr::S;
    const S m = op == MX_OP_MAX ? BinOp<DT, MX_OP_MAX>::apply(a, b) : BinOp<DT, MX_OP_MIN>::apply(a, b);
    const S mb = BinOp<DT, MX_OP_EQ>::apply(b, m);
    const S mask = side ? mb : BinOp<DT, MX_OP_SUB>::apply(Tr::st(1.0f), mb);
    return BinOp<DT, MX_OP_MUL>::apply(g, mask);
}

// One VEC-wide slot of R (and of G, which has R's strides) per thread; av / bv: the operand's
// innermost stride is 1 (else 0: one value repeated across the slot).
template <int DT, int VEC>
__global__ __launch_bounds__(kBlock) void max_grad_vec_kernel(
    typename dt_traits<DT>::S* __restrict__ R, const typename dt_traits<DT>::S* __restrict__ A,
    const typename dt_traits<DT>::S* __restrict__ B, const typename dt_traits<DT>::S* __restrict__ G,
    uint32_t nvec, FastDiv inner_vecs, OuterDesc od, int av, int bv, int op, int side) {
    using S = typename dt_traits<DT>::S;
    using V = Vec<S, VEC>;
    const uint32_t v = blockIdx.x * kBlock + threadIdx.x;
    if (v >= nvec) return;
    uint32_t row = inner_vecs.div(v);
    const uint32_t col = (v - row * inner_vecs.d) * VEC;
    uint64_t oa = 0, ob = 0, orr = 0;
    for (int d = od.n - 1; d >= 0; --d) {
        const uint32_t q = od.shape[d].div(row);
        const uint32_t idx = row - q * od.shape[d].d;
        row = q;
        oa += (uint64_t)idx * od.sA[d];
        ob += (uint64_t)idx * od.sB[d];
        orr += (uint64_t)idx * od.sR[d];
    }
    V va, vb;
    if (av) va = *reinterpret_cast<const V*>(A + oa + col);
    else {
        const S x = A[oa];
#pragma unroll
        for (int i = 0; i < VEC; i++) va.v[i] = x;
    }
    if (bv) vb = *reinterpret_cast<const V*>(B + ob + col);
    else {
        const S x = B[ob];
#pragma unroll
        for (int i = 0; i < VEC; i++) vb.v[i] = x;
    }
    const V vg = *reinterpret_cast<const V*>(G + orr + col);
    V r;
#pragma unroll
    for (int i = 0; i < VEC; i++) r.v[i] = max_grad_elem<DT>(va.v[i], vb.v[i], vg.v[i], op, side);
    *reinterpret_cast<V*>(R + orr + col) = r;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void max_grad_scalar_kernel(
    typename dt_traits<DT>::S* __restrict__ R, const typename dt_traits<DT>::S* __restrict__ A,
    const typename dt_traits<DT>::S* __restrict__ B, const typename dt_traits<DT>::S* __restrict__ G,
    uint32_t total, FullDesc fd, int op, int side) {
    const uint32_t g = blockIdx.x * kBlock + threadIdx.x;
    if (g >= total) return;
    uint32_t rem = g;
    uint64_t oa = 0, ob = 0, orr = 0;
    for (int d = fd.n - 1; d >= 0; --d) {
        const uint32_t q = fd.shape[d].div(rem);
        const uint32_t idx = rem - q * fd.shape[d].d;
        rem = q;
        oa += (uint64_t)idx * fd.sA[d];
        ob += (uint64_t)idx * fd.sB[d];
        orr += (uint64_t)idx * fd.sR[d];
    }
    R[orr] = max_grad_elem<DT>(A[oa], B[ob], G[orr], op, side);
}

template <int DT>
int launch_max_grad(int op, int side, int cdims, const uint32_t* shape, const uint32_t* sR, const uint32_t* sA,
                    const uint32_t* sB, void* Rp, const void* Ap, const void* Bp, const void* Gp, uint64_t total,
                    hipStream_t st) {
    using S = typename dt_traits<DT>::S;
    constexpr int VEC = 16 / sizeof(S);
    S* R = (S*)Rp;
    const S* A = (const S*)Ap;
    const S* B = (const S*)Bp;
    const S* G = (const S*)Gp;
    const int in = cdims - 1;
    bool vec = cdims > 0 && sR[in] == 1 && sA[in] <= 1 && sB[in] <= 1 && shape[in] % VEC == 0 &&
               (uintptr_t)R % 16 == 0 && (uintptr_t)G % 16 == 0 && (sA[in] == 0 || (uintptr_t)A % 16 == 0) &&
               (sB[in] == 0 || (uintptr_t)B % 16 == 0);
    for (int d = 0; vec && d < in; d++)
        if (sR[d] % VEC || (sA[in] == 1 && sA[d] % VEC) || (sB[in] == 1 && sB[d] % VEC)) vec = false;
    if (vec) {
        OuterDesc od{};
        od.n = in;
        for (int d = 0; d < in; d++) {
            od.shape[d] = FastDiv(shape[d]);
            od.sA[d] = sA[d]; od.sB[d] = sB[d]; od.sR[d] = sR[d];
        }
        const uint32_t nvec = (uint32_t)(total / VEC);
        hipLaunchKernelGGL((max_grad_vec_kernel<DT, VEC>), dim3((nvec + kBlock - 1) / kBlock), dim3(kBlock), 0, st, R,
                           A, B, G, nvec, FastDiv(shape[in] / VEC), od, (int)sA[in], (int)sB[in], op, side);
    } else {
        FullDesc fd{};
        fd.n = cdims;
        for (int d = 0; d < cdims; d++) {
            fd.shape[d] = FastDiv(shape[d]);
            fd.sA[d] = sA[d]; fd.sB[d] = sB[d]; fd.sR[d] = sR[d];
        }
        hipLaunchKernelGGL((max_grad_scalar_kernel<DT>), dim3((uint32_t)((total + kBlock - 1) / kBlock)), dim3(kBlock),
                           0, st, R, A, B, G, (uint32_t)total, fd, op, side);
    }
    MX_HIP(hipGetLastError());
    return MX_OK;
}

template <int DT, int OP>
int launch_typed(int cdims, const uint32_t* shape, const uint32_t* sR, const uint32_t* sA,
                 const uint32_t* sB, void* Rp, const void* Ap, const void* Bp, uint64_t total,
                 hipStream_t st) {
    using S = typename dt_traits<DT>::S;
    S* R = (S*)Rp;
    const S* A = (const S*)Ap;
    const S* B = (const S*)Bp;
    constexpr int VEC = 16 / sizeof(S);
    if (cdims == 0) {
        FullDesc fd{};
        fd.n = 0;
        hipLaunchKernelGGL((bcast_scalar_kernel<DT, OP>), dim3(1), dim3(kBlock), 0, st, R, A, B, 1u, fd);
        MX_HIP(hipGetLastError());
        return MX_OK;
    }
    const int in = cdims - 1;
    const uint32_t inner = shape[in];
    bool vec = (VEC > 1) && sR[in] == 1 && (sA[in] <= 1) && (sB[in] <= 1) && (inner % VEC == 0) &&
               (sA[in] == 1 || sB[in] == 1) && ((uintptr_t)R % 16 == 0);
    if (vec && sA[in] == 1 && (uintptr_t)A % 16 != 0) vec = false;
    if (vec && sB[in] == 1 && (uintptr_t)B % 16 != 0) vec = false;
    for (int d = 0; vec && d < in; d++) {
        if (sR[d] % VEC) vec = false;
        if (sA[in] == 1 && sA[d] % VEC) vec = false;
        if (sB[in] == 1 && sB[d] % VEC) vec = false;
    }
    if (vec) {
        OuterDesc od{};
        od.n = in;
        for (int d = 0; d < in; d++) {
            od.shape[d] = FastDiv(shape[d]);
            od.sA[d] = sA[d]; od.sB[d] = sB[d]; od.sR[d] = sR[d];
        }
        uint32_t nvec = (uint32_t)(total / VEC);
        dim3 grid((nvec + kBlock * kUnroll - 1) / (kBlock * kUnroll));
        FastDiv iv(inner / VEC);
        // an operand that no axis broadcasts is read once: nontemporal loads
        bool sa = sA[in] == 1, sb = sB[in] == 1;
        for (int d = 0; d < in; d++) {
            if (shape[d] > 1 && sA[d] == 0) sa = false;
            if (shape[d] > 1 && sB[d] == 0) sb = false;
        }
        const int nt = (sa ? 1 : 0) | (sb ? 2 : 0);
        if (sA[in] == 1 && sB[in] == 1)
            hipLaunchKernelGGL((bcast_vec_kernel<DT, OP, VEC, true, true>), grid, dim3(kBlock), 0, st, R, A, B, nvec, iv, od, nt);
        else if (sA[in] == 1)
            hipLaunchKernelGGL((bcast_vec_kernel<DT, OP, VEC, true, false>), grid, dim3(kBlock), 0, st, R, A, B, nvec, iv, od, nt);
        else
            hipLaunchKernelGGL((bcast_vec_kernel<DT, OP, VEC, false, true>), grid, dim3(kBlock), 0, st, R, A, B, nvec, iv, od, nt);
    } else {
        FullDesc fd{};
        fd.n = cdims;
        for (int d = 0; d < cdims; d++) {
            fd.shape[d] = FastDiv(shape[d]);
            fd.sA[d] = sA[d]; fd.sB[d] = sB[d]; fd.sR[d] = sR[d];
        }
        dim3 grid((uint32_t)((total + kBlock - 1) / kBlock));
        hipLaunchKernelGGL((bcast_scalar_kernel<DT, OP>), grid, dim3(kBlock), 0, st, R, A, B, (uint32_t)total, fd);
    }
    MX_HIP(hipGetLastError());
    return MX_OK;
}

template <int DT>
int launch_op(int op, int cdims, const uint32_t* shape, const uint32_t* sR, const uint32_t* sA,
              const uint32_t* sB, void* R, const void* A, const void* B, uint64_t total, hipStream_t st) {
    switch (op) {
    case MX_OP_ADD: return launch_typed<DT, MX_OP_ADD>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    case MX_OP_SUB: return launch_typed<DT, MX_OP_SUB>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    case MX_OP_MUL: return launch_typed<DT, MX_OP_MUL>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    case MX_OP_DIV: return launch_typed<DT, MX_OP_DIV>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    case MX_OP_MAX: return launch_typed<DT, MX_OP_MAX>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    case MX_OP_MIN: return launch_typed<DT, MX_OP_MIN>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    case MX_OP_EQ: return launch_typed<DT, MX_OP_EQ>(cdims, shape, sR, sA, sB, R, A, B, total, st);
    default: return fail(MX_ERR_INVALID_ARG, "mx_launch_bcast_binary: unknown op " + std::to_string(op));
    }
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_launch_bcast_binary(int op, int dtype, int cdims, const uint32_t* shape,
                                      const uint32_t* sR, const uint32_t* sA, const uint32_t* sB,
                                      void* R, const void* A, const void* B, void* stream) {
    if (cdims < 0 || cdims > MX_MAX_DIMS)
        return fail(MX_ERR_INVALID_ARG, "mx_launch_bcast_binary: cdims " + std::to_string(cdims) + " outside [0, 8]");
    if (cdims > 0 && (!shape || !sR || !sA || !sB))
        return fail(MX_ERR_INVALID_ARG, "mx_launch_bcast_binary: null descriptor");
    if (op < MX_OP_ADD || op > MX_OP_EQ)
        return fail(MX_ERR_INVALID_ARG, "mx_launch_bcast_binary: unknown op " + std::to_string(op));
    uint64_t total = 1;
    for (int d = 0; d < cdims; d++) total *= shape[d];
    if (total == 0) return MX_OK;
    if (total > 0xffffffffull)
        return fail(MX_ERR_INVALID_ARG, "mx_launch_bcast_binary: more than 2^32-1 elements (size_m indexing)");
    if (!R || !A || !B) return fail(MX_ERR_INVALID_ARG, "mx_launch_bcast_binary: null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    if (dtype == MX_COMPLEX64) {
        switch (op) {
        case MX_OP_ADD: return launch_typed<MX_COMPLEX64, MX_OP_ADD>(cdims, shape, sR, sA, sB, R, A, B, total, st);
        case MX_OP_SUB: return launch_typed<MX_COMPLEX64, MX_OP_SUB>(cdims, shape, sR, sA, sB, R, A, B, total, st);
        case MX_OP_MUL: return launch_typed<MX_COMPLEX64, MX_OP_MUL>(cdims, shape, sR, sA, sB, R, A, B, total, st);
        case MX_OP_DIV: return launch_typed<MX_COMPLEX64, MX_OP_DIV>(cdims, shape, sR, sA, sB, R, A, B, total, st);
        default:
            return fail(MX_ERR_UNSUPPORTED, "mx_launch_bcast_binary: Complex64 has Add / Sub / Mul / Divide only (op " +
                                                std::to_string(op) + ")");
        }
    }
    int rc = MX_OK;
    bool ok = dispatch_dtype(dtype, [&](auto dt) {
        rc = launch_op<decltype(dt)::value>(op, cdims, shape, sR, sA, sB, R, A, B, total, st);
    });
    if (!ok)
        return fail(MX_ERR_UNSUPPORTED, "mx_launch_bcast_binary: no kernel for dtype " + std::to_string(dtype));
    return rc;
}

extern "C" int mx_launch_max_grad(int op, int side, int dtype, int cdims, const uint32_t* shape, const uint32_t* sR,
                                  const uint32_t* sA, const uint32_t* sB, void* R, const void* A, const void* B,
                                  const void* G, void* stream) {
    const char* who = "mx_launch_max_grad";
    if (op != MX_OP_MAX && op != MX_OP_MIN)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": op must be MX_OP_MAX or MX_OP_MIN");
    if (side != 0 && side != 1) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": side must be 0 (a) or 1 (b)");
    if (cdims < 0 || cdims > MX_MAX_DIMS)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": cdims " + std::to_string(cdims) + " outside [0, 8]");
    if (cdims > 0 && (!shape || !sR || !sA || !sB)) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null descriptor");
    uint64_t total = 1;
    for (int d = 0; d < cdims; d++) total *= shape[d];
    if (total == 0) return MX_OK;
    if (total > 0xffffffffull)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": more than 2^32-1 elements (size_m indexing)");
    if (!R || !A || !B || !G) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    switch (dtype) {
    case MX_FLOAT32: return launch_max_grad<MX_FLOAT32>(op, side, cdims, shape, sR, sA, sB, R, A, B, G, total, st);
    case MX_FLOAT16: return launch_max_grad<MX_FLOAT16>(op, side, cdims, shape, sR, sA, sB, R, A, B, G, total, st);
    case MX_BFLOAT16: return launch_max_grad<MX_BFLOAT16>(op, side, cdims, shape, sR, sA, sB, R, A, B, G, total, st);
    default:
        return fail(MX_ERR_UNSUPPORTED, std::string(who) + ": float32 / float16 / bfloat16 only, dtype " +
                                            std::to_string(dtype));
    }
}
