// copy.hip -- strided copy with dtype cast: dst[idx . sDst] = cast(src[idx . sSrc]).
//
// Replaces copyGPUinplace / copyGPUinplaceTypeCasted and the CopyInplaceGPU kernels
// (Matrix.mm:1699-1976, Copy.metal:14-80); the element semantics are those of the CPU copy
// (copyCPUinplace / copyCPUinplaceTypeCasted, matrix.h:1337-1550), whose dtype_cast
// (matrix.h:306-313) is a static_cast:
//   - float -> float goes through float (16-bit targets round to nearest even);
//   - integer -> float rounds to nearest even (64-bit integers included);
//   - float -> integer truncates toward zero and saturates (NaN -> 0): 8- and 16-bit targets
//     saturate to the 32-bit range first and then keep the low bits, as arm64's fcvtzs /
//     fcvtzu followed by a narrowing store do;
//   - integer -> integer keeps the low bits (two's complement);
//   - anything -> bool is (value != 0); bool reads as 0 / 1;
//   - a real dtype -> complex64 is complex64(float(value), 0), the complex64(float re, float im = 0)
//     constructor static_cast picks (complex.h:22); complex64 defines no conversion to a real type,
//     so complex64 -> real is rejected;
//   - a copy within one dtype moves the element's bits (the blit and CopyInplaceGPU_<t>_<t> of the
//     reference, static_cast<T>(T)), complex64 included.
//
// Layout: the iteration space is a collapsed descriptor (any cdims <= 8).  Same-dtype copies
// whose innermost axis is unit-stride on both sides move 16 bytes per thread; same-dtype
// transposes (16-byte aligned) move 16-byte register blocks; everything else runs one element
// per thread with FastDiv index decomposition.
#include "common.hpp"

namespace mx {
namespace {

// A source element widened to one of three carriers, as the cast needs it.
struct Wide {
    int kind;            // 0 float, 1 signed integer, 2 unsigned integer
    float f;
    int64_t i;
    uint64_t u;
};

template <int SD>
__device__ __forceinline__ Wide widen(typename dt_traits<SD>::S x) {
    Wide w{0, 0.0f, 0, 0};
    if constexpr (dt_traits<SD>::is_float) {
        w.kind = 0;
        w.f = dt_traits<SD>::ld(x);
    } else if constexpr (SD == MX_BOOL) {
        w.kind = 2;
        w.u = x != 0;
    } else if constexpr (dt_traits<SD>::is_signed) {
        w.kind = 1;
        w.i = (int64_t)x;
    } else {
        w.kind = 2;
        w.u = (uint64_t)x;
    }
    return w;
}

__device__ __forceinline__ int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
__device__ __forceinline__ uint32_t sat_u32(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 4294967296.0f) return UINT32_MAX;
    return (uint32_t)v;
}
__device__ __forceinline__ int64_t sat_i64(float v) {
    if (v != v) return 0;
    if (v >= 9.2233720368547758e18f) return INT64_MAX;
    if (v <= -9.2233720368547758e18f) return INT64_MIN;
    return (int64_t)v;
}
__device__ __forceinline__ uint64_t sat_u64(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 1.8446744073709552e19f) return UINT64_MAX;
    return (uint64_t)v;
}

template <int DD>
__device__ __forceinline__ typename dt_traits<DD>::S narrow(const Wide& w) {
    using Tr = dt_traits<DD>;
    using S = typename Tr::S;
    if constexpr (DD == MX_COMPLEX64) {
        return c64{w.kind == 0 ? w.f : (w.kind == 1 ? (float)w.i : (float)w.u), 0.0f};
    } else if constexpr (Tr::is_float) {
        const float v = w.kind == 0 ? w.f : (w.kind == 1 ? (float)w.i : (float)w.u);
        return Tr::st(v);
    } else if constexpr (DD == MX_BOOL) {
        return (S)(w.kind == 0 ? (w.f != 0.0f) : ((w.kind == 1 ? (uint64_t)w.i : w.u) != 0));
    } else {
        const int64_t iv = w.kind == 1 ? w.i : (int64_t)w.u;       // integer sources
        const uint64_t uv = (uint64_t)iv;
        if constexpr (DD == MX_INT64) return w.kind == 0 ? sat_i64(w.f) : iv;
        else if constexpr (DD == MX_UINT64) return w.kind == 0 ? sat_u64(w.f) : uv;
        else if constexpr (Tr::is_signed) return w.kind == 0 ? (S)sat_i32(w.f) : (S)iv;
        else return w.kind == 0 ? (S)sat_u32(w.f) : (S)uv;
    }
}

struct CopyDesc {
    int n;
    FastDiv shape[MX_MAX_DIMS];
    uint32_t sd[MX_MAX_DIMS], ss[MX_MAX_DIMS];
};

template <int DD, int SD>
__global__ __launch_bounds__(256) void copy_scalar_kernel(typename dt_traits<DD>::S* __restrict__ dst,
                                                          const typename dt_traits<SD>::S* __restrict__ src,
                                                          uint64_t total, CopyDesc d) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x; g < total; g += stride) {
        uint64_t od = 0, os = 0;
        if (g < 0x100000000ull) {                // 32-bit decomposition (every shape axis < 2^32)
            uint32_t rem = (uint32_t)g;
            for (int k = d.n - 1; k >= 0; --k) {
                const uint32_t q = d.shape[k].div(rem);
                const uint32_t idx = rem - q * d.shape[k].d;
                rem = q;
                od += (uint64_t)idx * d.sd[k];
                os += (uint64_t)idx * d.ss[k];
            }
        } else {
            uint64_t rem = g;
            for (int k = d.n - 1; k >= 0; --k) {
                const uint64_t idx = rem % d.shape[k].d;
                rem /= d.shape[k].d;
                od += idx * d.sd[k];
                os += idx * d.ss[k];
            }
        }
        dst[od] = narrow<DD>(widen<SD>(src[os]));
    }
}

// Same dtype, innermost axis contiguous on both sides and a multiple of the 16-byte vector:
// each thread moves one 16-byte chunk; the outer axes decompose the chunk's row.
struct RowDesc {
    int n;                                  // outer axes
    FastDiv shape[MX_MAX_DIMS];
    uint32_t sd[MX_MAX_DIMS], ss[MX_MAX_DIMS];
    FastDiv row_chunks;                     // 16-byte chunks per innermost row
};

__global__ __launch_bounds__(256) void copy_rows16_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                          uint64_t chunks, uint32_t elem_bytes, RowDesc d) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x; g < chunks; g += stride) {
        const uint32_t gg = (uint32_t)g;                 // launcher keeps chunks < 2^32
        uint32_t row = d.row_chunks.div(gg);
        const uint32_t c = gg - row * d.row_chunks.d;
        uint64_t od = 0, os = 0;                          // element offsets of the row start
        for (int k = d.n - 1; k >= 0; --k) {
            const uint32_t q = d.shape[k].div(row);
            const uint32_t idx = row - q * d.shape[k].d;
            row = q;
            od += (uint64_t)idx * d.sd[k];
            os += (uint64_t)idx * d.ss[k];
        }
        const uint32_t per = 16 / elem_bytes;
        dst[od / per + c] = src[os / per + c];
    }
}

// Same dtype, a transpose: the destination's innermost axis l is strided in the source while
// another axis j is unit-stride there (a transposed view made contiguous, as dot() does with
// B^T).  The (j, l) plane is copied in VE x VE register blocks (VE = elements per 16 bytes):
// lane (lb = lane % 8, jb = lane / 8) of wave w loads VE source rows (l .. l + VE - 1) of VE
// consecutive j, transposes the block in registers and stores VE destination rows (j ..) of VE
// consecutive l, so 8 lanes cover 128 contiguous bytes on both sides.  Further axes are the
// batch (blockIdx.z).  Extents, strides and pointers are whole 16-byte units on this path.
struct TransDesc {
    int nb;                                 // batch axes
    FastDiv bshape[MX_MAX_DIMS];
    uint32_t bsd[MX_MAX_DIMS], bss[MX_MAX_DIMS];
    uint32_t J, L;                          // plane extents: source-contiguous j, destination-contiguous l
    uint32_t sdj, ssl;                      // destination stride of j, source stride of l
};

template <typename S>
__global__ __launch_bounds__(256) void copy_transpose16_kernel(S* __restrict__ dst, const S* __restrict__ src,
                                                               TransDesc d) {
    constexpr int VE = 16 / sizeof(S);
    struct alignas(16) V { S v[VE]; };
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t l = blockIdx.y * (8 * VE) + (lane & 7) * VE;
    const uint32_t j = (blockIdx.x * 32 + wave * 8 + (lane >> 3)) * VE;
    if (j >= d.J || l >= d.L) return;
    uint32_t b = blockIdx.z;
    uint64_t od = 0, os = 0;
    for (int k = d.nb - 1; k >= 0; --k) {
        const uint32_t q = d.bshape[k].div(b);
        const uint32_t idx = b - q * d.bshape[k].d;
        b = q;
        od += (uint64_t)idx * d.bsd[k];
        os += (uint64_t)idx * d.bss[k];
    }
    const S* s0 = src + os + j;
    V v[VE];
#pragma unroll
    for (int i = 0; i < VE; i++) v[i] = *reinterpret_cast<const V*>(s0 + (uint64_t)(l + i) * d.ssl);
    S* d0 = dst + od + l;
#pragma unroll
    for (int jj = 0; jj < VE; jj++) {
        V w;
#pragma unroll
        for (int i = 0; i < VE; i++) w.v[i] = v[i].v[jj];
        *reinterpret_cast<V*>(d0 + (uint64_t)(j + jj) * d.sdj) = w;
    }
}

// Sets up the transpose path; false when the copy is not a same-dtype aligned transpose.
template <typename S>
bool launch_transpose16(int cdims, const uint32_t* shape, const uint32_t* sDst, const uint32_t* sSrc, void* dst,
                        const void* src, hipStream_t st) {
    constexpr uint32_t VE = 16 / sizeof(S);
    const int last = cdims - 1;
    if (cdims < 2 || sDst[last] != 1 || sSrc[last] == 1) return false;
    int jax = -1;
    for (int k = last - 1; k >= 0; --k)
        if (sSrc[k] == 1 && shape[k] > 1) { jax = k; break; }
    if (jax < 0) return false;
    if ((uintptr_t)dst % 16 || (uintptr_t)src % 16) return false;
    TransDesc d{};
    d.J = shape[jax];
    d.L = shape[last];
    d.sdj = sDst[jax];
    d.ssl = sSrc[last];
    if (d.J % VE || d.L % VE || d.sdj % VE || d.ssl % VE) return false;
    uint64_t batch = 1;
    for (int k = 0; k < last; k++) {
        if (k == jax) continue;
        if (sDst[k] % VE || sSrc[k] % VE) return false;
        d.bshape[d.nb] = FastDiv(shape[k]);
        d.bsd[d.nb] = sDst[k];
        d.bss[d.nb] = sSrc[k];
        d.nb++;
        batch *= shape[k];
    }
    if (batch > 65535) return false;
    const dim3 grid((d.J + 32 * VE - 1) / (32 * VE), (d.L + 8 * VE - 1) / (8 * VE), (uint32_t)batch);
    hipLaunchKernelGGL((copy_transpose16_kernel<S>), grid, dim3(256), 0, st, (S*)dst, (const S*)src, d);
    return true;
}

template <typename F>
bool dispatch_pair(int dd, int sd, F&& f) {
    bool ok = false;
    dispatch_dtype(dd, [&](auto D) {
        ok = dispatch_dtype(sd, [&](auto S) { f(D, S); });
    });
    return ok;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_launch_copy_strided(int dst_dtype, int src_dtype, int cdims, const uint32_t* shape,
                                      const uint32_t* sDst, const uint32_t* sSrc, void* dst, const void* src,
                                      void* stream) {
    if (cdims < 0 || cdims > MX_MAX_DIMS)
        return fail(MX_ERR_INVALID_ARG, "mx_launch_copy_strided: cdims " + std::to_string(cdims) + " outside [0, 8]");
    if (cdims > 0 && (!shape || !sDst || !sSrc)) return fail(MX_ERR_INVALID_ARG, "mx_launch_copy_strided: null descriptor");
    if (dtype_size(dst_dtype) == 0 || dtype_size(src_dtype) == 0)
        return fail(MX_ERR_UNSUPPORTED, "mx_launch_copy_strided: no kernel for dtypes " + std::to_string(dst_dtype) +
                                            " <- " + std::to_string(src_dtype));
    if (src_dtype == MX_COMPLEX64 && dst_dtype != MX_COMPLEX64)
        return fail(MX_ERR_UNSUPPORTED, "mx_launch_copy_strided: Complex64 has no cast to a real dtype (" +
                                            std::to_string(dst_dtype) + ")");
    uint64_t total = 1;
    for (int k = 0; k < cdims; k++) total *= shape[k];
    if (total == 0) return MX_OK;
    if (!dst || !src) return fail(MX_ERR_INVALID_ARG, "mx_launch_copy_strided: null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;

    const size_t es = dtype_size(dst_dtype);
    // 16-byte row path
    if (dst_dtype == src_dtype && cdims >= 1 && sDst[cdims - 1] == 1 && sSrc[cdims - 1] == 1 &&
        (shape[cdims - 1] * es) % 16 == 0 && (uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0) {
        const uint32_t per = (uint32_t)(16 / es);
        bool aligned = true;
        RowDesc d{};
        d.n = cdims - 1;
        for (int k = 0; k < cdims - 1; k++) {
            d.shape[k] = FastDiv(shape[k]);
            d.sd[k] = sDst[k];
            d.ss[k] = sSrc[k];
            if (sDst[k] % per || sSrc[k] % per) aligned = false;
        }
        const uint64_t chunks = total / per;
        if (aligned && chunks < 0xffffffffull) {
            d.row_chunks = FastDiv(shape[cdims - 1] / per);
            const uint64_t want = (chunks + 255) / 256;
            const uint32_t blocks = (uint32_t)(want < 65536 ? want : 65536);
            hipLaunchKernelGGL(copy_rows16_kernel, dim3(blocks), dim3(256), 0, st, (uint4*)dst, (const uint4*)src,
                               chunks, (uint32_t)es, d);
            MX_HIP(hipGetLastError());
            return MX_OK;
        }
    }
    if (dst_dtype == src_dtype) {
        bool done = false;
        if (es == 4) done = launch_transpose16<uint32_t>(cdims, shape, sDst, sSrc, dst, src, st);
        else if (es == 2) done = launch_transpose16<uint16_t>(cdims, shape, sDst, sSrc, dst, src, st);
        else if (es == 8) done = launch_transpose16<uint64_t>(cdims, shape, sDst, sSrc, dst, src, st);
        if (done) {
            MX_HIP(hipGetLastError());
            return MX_OK;
        }
    }
    CopyDesc d{};
    d.n = cdims;
    for (int k = 0; k < cdims; k++) {
        d.shape[k] = FastDiv(shape[k]);
        d.sd[k] = sDst[k];
        d.ss[k] = sSrc[k];
    }
    const uint64_t want = (total + 255) / 256;
    const uint32_t blocks = (uint32_t)(want < 65536 ? want : 65536);
    int rc = MX_OK;
    auto launch = [&](auto D, auto S) {
        constexpr int DD = decltype(D)::value, SD = decltype(S)::value;
        hipLaunchKernelGGL((copy_scalar_kernel<DD, SD>), dim3(blocks), dim3(256), 0, st,
                           (typename dt_traits<DD>::S*)dst, (const typename dt_traits<SD>::S*)src, total, d);
        if (hipGetLastError() != hipSuccess) rc = fail(MX_ERR_HIP, "mx_launch_copy_strided: launch failed");
    };
    if (dst_dtype == src_dtype) {                  // bits, through the unsigned carrier of the element size
        switch (es) {
        case 1: launch(std::integral_constant<int, MX_UINT8>{}, std::integral_constant<int, MX_UINT8>{}); break;
        case 2: launch(std::integral_constant<int, MX_UINT16>{}, std::integral_constant<int, MX_UINT16>{}); break;
        case 4: launch(std::integral_constant<int, MX_UINT32>{}, std::integral_constant<int, MX_UINT32>{}); break;
        default: launch(std::integral_constant<int, MX_UINT64>{}, std::integral_constant<int, MX_UINT64>{}); break;
        }
        return rc;
    }
    if (dst_dtype == MX_COMPLEX64) {
        if (!dispatch_dtype(src_dtype, [&](auto S) { launch(std::integral_constant<int, MX_COMPLEX64>{}, S); }))
            return fail(MX_ERR_UNSUPPORTED, "mx_launch_copy_strided: no kernel for dtype " + std::to_string(src_dtype));
        return rc;
    }
    dispatch_pair(dst_dtype, src_dtype, launch);
    return rc;
}
