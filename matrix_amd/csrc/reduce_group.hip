// reduce_group.hip -- mx_launch_reduce_group: several independent reductions of one dtype over one
// collapsed descriptor.  Float dtypes run as one launch of the group kernels (reduce_group_impl.hpp,
// instantiated per dtype in reduce_group_f32 / _f16 / _bf16.hip); the other dtypes run each member
// through mx_launch_reduce.
#include "reduce_plans.hpp"

namespace mx {
template <int DT>
int run_reduce_group(const Desc& d, int n, const int* ops, void* const* outs, const void* const* ins, void* const* ws,
                     const size_t* ws_bytes, hipStream_t st);
}  // namespace mx

using namespace mx;

extern "C" int mx_launch_reduce_group(int n, const int* ops, int dtype, uint32_t reduce_stride, uint32_t n_reduce,
                                      int cdims, const uint32_t* shape, const uint32_t* sOut, const uint32_t* sIn,
                                      void* const* outs, const void* const* ins, void* const* workspaces,
                                      const size_t* workspace_bytes, void* stream) {
    const char* who = "mx_launch_reduce_group";
    if (n < 0 || n > MX_REDUCE_GROUP_MAX)
        return fail(MX_ERR_INVALID_ARG, std::string(who) + ": group of " + std::to_string(n) + " (at most " +
                                            std::to_string(MX_REDUCE_GROUP_MAX) + ")");
    if (n == 0) return MX_OK;
    if (!ops || !outs || !ins) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null array");
    Desc d;
    for (int k = 0; k < n; k++) {
        int rc = check_desc(who, ops[k], cdims, shape, sOut, sIn, reduce_stride, n_reduce, &d);
        if (rc != MX_OK) return rc;
    }
    uint64_t tot = 1;
    for (int i = 0; i < d.cd; i++) tot *= d.shape[i];
    if (tot == 0) return MX_OK;
    for (int k = 0; k < n; k++)
        if (!outs[k] || (!ins[k] && n_reduce > 0)) return fail(MX_ERR_INVALID_ARG, std::string(who) + ": null buffer");
    hipStream_t st;
    if (!resolve_stream(stream, &st)) return MX_ERR_NOT_INITIALIZED;
    int rc = MX_OK;
    // the float types run as one group launch; the others as one launch per member
    bool ok = dispatch_dtype(dtype, [&](auto dt) {
        constexpr int DT = decltype(dt)::value;
        if constexpr (DT == MX_FLOAT32 || DT == MX_FLOAT16 || DT == MX_BFLOAT16) {
            rc = run_reduce_group<DT>(d, n, ops, outs, ins, workspaces, workspace_bytes, st);
        } else {
            for (int k = 0; k < n && rc == MX_OK; k++)
                rc = mx_launch_reduce(ops[k], dtype, reduce_stride, n_reduce, cdims, shape, sOut, sIn, outs[k], ins[k],
                                      workspaces ? workspaces[k] : nullptr, workspace_bytes ? workspace_bytes[k] : 0, st);
        }
    });
    if (!ok) return fail(MX_ERR_UNSUPPORTED, std::string(who) + ": no kernel for dtype " + std::to_string(dtype));
    return rc;
}
