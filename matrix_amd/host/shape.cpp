// shape.cpp -- broadcast and dim-collapse helpers (host only).
//
// These produce the collapsed shape / stride descriptors the kernels consume, with the
// same merge rules as the reference so that a graph builds the same iteration space:
//   collapse (Mods/Utils.mm:114-202)          axis 0 always opens a slot; later size-1 axes
//                                             are dropped; axis i merges into the open slot
//                                             when every operand's stride there equals
//                                             stride[i] * shape[i] and the merged extent
//                                             stays <= size_cap; the inner stride wins.
//   collapse_matmul (Mods/Utils.mm:204-252)   the same over batch axes only; the last two
//                                             axes are appended verbatim.
//   collapse_reduce (Mods/Utils.mm:321-376)   the reduced axis is a hard split (kept as its
//                                             own slot only with keep_dims); with
//                                             outer_collapsed the output has one axis fewer,
//                                             so its stride index shifts down after the axis.
//   broadcast (Matrix.mm:161-331)             right-aligned, size-1 axes get stride 0,
//                                             missing leading axes stride 0, contiguous out.
#include "../../include/matrix_amd.h"
#include "../../include/matrix_amd_shape.h"

#include <array>
#include <cstring>
#include <string>

namespace mx {
void set_error(const std::string& msg);
}

namespace {

constexpr int kMax = MX_MAX_DIMS;

template <int K>
struct Collapsed {
    uint32_t shape[kMax];
    uint32_t s[K][kMax];
    uint32_t dims = 0;
};

// Generic collapse over K stride sets for axes [begin, end) after the seeded axis 0.
template <int K>
void collapse_into(Collapsed<K>& r, const uint32_t* shape, const uint32_t* const* strides,
                   uint32_t begin, uint32_t end, uint64_t cap) {
    uint32_t slot = r.dims - 1;
    for (uint32_t i = begin; i < end; i++) {
        if (shape[i] == 1) continue;
        bool merge = (uint64_t)r.shape[slot] * shape[i] <= cap;
        for (int k = 0; merge && k < K; k++)
            merge = (uint64_t)r.s[k][slot] == (uint64_t)strides[k][i] * shape[i];
        if (!merge) {
            slot++;
            r.shape[slot] = shape[i];
        } else {
            r.shape[slot] *= shape[i];
        }
        for (int k = 0; k < K; k++) r.s[k][slot] = strides[k][i];
    }
    r.dims = slot + 1;
}

template <int K>
Collapsed<K> collapse(const uint32_t* shape, const uint32_t* const* strides, uint32_t dims, uint64_t cap) {
    Collapsed<K> r{};
    if (dims == 0) return r;
    r.shape[0] = shape[0];
    for (int k = 0; k < K; k++) r.s[k][0] = strides[k][0];
    r.dims = 1;
    collapse_into<K>(r, shape, strides, 1, dims, cap);
    return r;
}

int bad(const std::string& m) {
    mx::set_error(m);
    return MX_ERR_INVALID_ARG;
}

bool check_rank(uint32_t dims, const char* who) {
    if (dims > kMax) {
        mx::set_error(std::string(who) + ": rank above 8 (MAX_TENSOR_DIMS)");
        return false;
    }
    return true;
}

}  // namespace

extern "C" {

int mx_collapse_dims3(const uint32_t* shape, const uint32_t* sA, const uint32_t* sB,
                      const uint32_t* sC, uint32_t dims, uint64_t size_cap,
                      uint32_t* out_shape, uint32_t* out_sA, uint32_t* out_sB,
                      uint32_t* out_sC, uint32_t* out_dims) {
    if (!check_rank(dims, "mx_collapse_dims3")) return MX_ERR_INVALID_ARG;
    const uint32_t* st[3] = {sA, sB, sC};
    auto r = collapse<3>(shape, st, dims, size_cap);
    std::memcpy(out_shape, r.shape, sizeof(uint32_t) * r.dims);
    std::memcpy(out_sA, r.s[0], sizeof(uint32_t) * r.dims);
    std::memcpy(out_sB, r.s[1], sizeof(uint32_t) * r.dims);
    std::memcpy(out_sC, r.s[2], sizeof(uint32_t) * r.dims);
    *out_dims = r.dims;
    return MX_OK;
}

int mx_collapse_dims2(const uint32_t* shape, const uint32_t* sA, const uint32_t* sB,
                      uint32_t dims, uint64_t size_cap, uint32_t* out_shape,
                      uint32_t* out_sA, uint32_t* out_sB, uint32_t* out_dims) {
    if (!check_rank(dims, "mx_collapse_dims2")) return MX_ERR_INVALID_ARG;
    const uint32_t* st[2] = {sA, sB};
    auto r = collapse<2>(shape, st, dims, size_cap);
    std::memcpy(out_shape, r.shape, sizeof(uint32_t) * r.dims);
    std::memcpy(out_sA, r.s[0], sizeof(uint32_t) * r.dims);
    std::memcpy(out_sB, r.s[1], sizeof(uint32_t) * r.dims);
    *out_dims = r.dims;
    return MX_OK;
}

int mx_collapse_dims_matmul(const uint32_t* shape, const uint32_t* sA, const uint32_t* sB,
                            const uint32_t* sC, uint32_t dims, uint64_t size_cap,
                            uint32_t* out_shape, uint32_t* out_sA, uint32_t* out_sB,
                            uint32_t* out_sC, uint32_t* out_dims) {
    if (!check_rank(dims, "mx_collapse_dims_matmul")) return MX_ERR_INVALID_ARG;
    if (dims < 3) return bad("mx_collapse_dims_matmul: rank below 3 (rank-2 products use [M, N] directly)");
    const uint32_t* st[3] = {sA, sB, sC};
    Collapsed<3> r{};
    r.shape[0] = shape[0];
    for (int k = 0; k < 3; k++) r.s[k][0] = st[k][0];
    r.dims = 1;
    collapse_into<3>(r, shape, st, 1, dims - 2, size_cap);
    uint32_t nd = r.dims + 2;
    if (nd > kMax) return bad("mx_collapse_dims_matmul: collapsed rank above 8");
    for (int t = 0; t < 2; t++) {
        r.shape[nd - 2 + t] = shape[dims - 2 + t];
        for (int k = 0; k < 3; k++) r.s[k][nd - 2 + t] = st[k][dims - 2 + t];
    }
    std::memcpy(out_shape, r.shape, sizeof(uint32_t) * nd);
    std::memcpy(out_sA, r.s[0], sizeof(uint32_t) * nd);
    std::memcpy(out_sB, r.s[1], sizeof(uint32_t) * nd);
    std::memcpy(out_sC, r.s[2], sizeof(uint32_t) * nd);
    *out_dims = nd;
    return MX_OK;
}

int mx_collapse_dims_reduce2(const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                             uint32_t dims, int axis, int keep_dims, int outer_collapsed,
                             uint64_t size_cap, uint32_t* out_shape, uint32_t* out_sOut,
                             uint32_t* out_sIn, uint32_t* out_dims) {
    if (!check_rank(dims, "mx_collapse_dims_reduce2")) return MX_ERR_INVALID_ARG;
    int slot = -1;
    bool split = false;      // the next kept axis must open a new slot
    for (int i = 0; i < (int)dims; i++) {
        if (i == axis) {
            if (keep_dims) {
                slot++;
                out_shape[slot] = shape[i];
                out_sOut[slot] = sOut[i];
                out_sIn[slot] = sIn[i];
            }
            split = true;
            continue;
        }
        if (shape[i] == 1) continue;
        const int oi = (outer_collapsed && axis < i) ? i - 1 : i;
        const bool merge = !split && slot >= 0 &&
                           (uint64_t)out_sOut[slot] == (uint64_t)sOut[oi] * shape[i] &&
                           (uint64_t)out_sIn[slot] == (uint64_t)sIn[i] * shape[i] &&
                           (uint64_t)out_shape[slot] * shape[i] <= size_cap;
        if (merge) {
            out_shape[slot] *= shape[i];
        } else {
            slot++;
            out_shape[slot] = shape[i];
            split = false;
        }
        out_sOut[slot] = sOut[oi];
        out_sIn[slot] = sIn[i];
    }
    *out_dims = (uint32_t)(slot + 1);
    return MX_OK;
}

static int broadcast_common(bool matmul, const uint32_t* shape1, const uint32_t* strides1, uint32_t d1,
                            const uint32_t* shape2, const uint32_t* strides2, uint32_t d2,
                            uint32_t* out_shape, uint32_t* out_strides,
                            uint32_t* b1_shape, uint32_t* b1_strides,
                            uint32_t* b2_shape, uint32_t* b2_strides) {
    const uint32_t nd = d1 > d2 ? d1 : d2;
    if (nd > kMax) return bad("broadcast: rank above 8");
    if (matmul) {
        if (d1 < 2 || d2 < 2)
            return bad("ValueError: matmul: Input operand does not have enough dimensions (has to be >= 2)");
        if (shape1[d1 - 1] != shape2[d2 - 1])
            return bad("ValueError: matmul: Input operand 1 has a mismatch in its core dimension 0 (size " +
                       std::to_string(shape2[d2 - 1]) + " is different from " + std::to_string(shape1[d1 - 1]) + ")");
    }
    // right-align both operands; missing leading axes get stride 0
    for (uint32_t i = 0; i < nd; i++) {
        const int j1 = (int)i - (int)(nd - d1), j2 = (int)i - (int)(nd - d2);
        b1_shape[i] = j1 >= 0 ? shape1[j1] : 0;
        b1_strides[i] = j1 >= 0 ? strides1[j1] : 0;
        b2_shape[i] = j2 >= 0 ? shape2[j2] : 0;
        b2_strides[i] = j2 >= 0 ? strides2[j2] : 0;
    }
    const uint32_t first_core = matmul ? nd - 2 : nd;
    for (uint32_t i = 0; i < first_core; i++) {
        const bool has1 = i >= nd - d1, has2 = i >= nd - d2;
        if (!has1) { b1_shape[i] = b2_shape[i]; out_shape[i] = b2_shape[i]; continue; }
        if (!has2) { b2_shape[i] = b1_shape[i]; out_shape[i] = b1_shape[i]; continue; }
        if (b1_shape[i] == b2_shape[i]) { out_shape[i] = b1_shape[i]; continue; }
        if (b1_shape[i] == 1) {
            b1_shape[i] = b2_shape[i]; b1_strides[i] = 0; out_shape[i] = b2_shape[i];
        } else if (b2_shape[i] == 1) {
            b2_shape[i] = b1_shape[i]; b2_strides[i] = 0; out_shape[i] = b1_shape[i];
        } else {
            return bad("MatrixH: Incompatible shapes for broadcasting");
        }
    }
    if (matmul) {
        out_shape[nd - 2] = shape1[d1 - 2];   // M
        out_shape[nd - 1] = shape2[d2 - 2];   // N
    }
    uint32_t acc = 1;
    for (int i = (int)nd - 1; i >= 0; i--) {
        out_strides[i] = acc;
        acc *= out_shape[i];
    }
    return MX_OK;
}

int mx_broadcast_shapes(const uint32_t* shape1, const uint32_t* strides1, uint32_t d1,
                        const uint32_t* shape2, const uint32_t* strides2, uint32_t d2,
                        uint32_t* out_shape, uint32_t* out_strides,
                        uint32_t* b1_shape, uint32_t* b1_strides,
                        uint32_t* b2_shape, uint32_t* b2_strides) {
    return broadcast_common(false, shape1, strides1, d1, shape2, strides2, d2, out_shape, out_strides,
                            b1_shape, b1_strides, b2_shape, b2_strides);
}

int mx_broadcast_shapes_matmul(const uint32_t* shape1, const uint32_t* strides1, uint32_t d1,
                               const uint32_t* shape2, const uint32_t* strides2, uint32_t d2,
                               uint32_t* out_shape, uint32_t* out_strides,
                               uint32_t* b1_shape, uint32_t* b1_strides,
                               uint32_t* b2_shape, uint32_t* b2_strides) {
    return broadcast_common(true, shape1, strides1, d1, shape2, strides2, d2, out_shape, out_strides,
                            b1_shape, b1_strides, b2_shape, b2_strides);
}

}  // extern "C"
