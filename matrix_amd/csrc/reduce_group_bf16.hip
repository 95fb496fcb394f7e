// reduce_group_bf16.hip -- the bf16 instantiation of the reduction group launcher.
#include "reduce_group_impl.hpp"

template int mx::run_reduce_group<MX_BFLOAT16>(const Desc& d, int n, const int* ops, void* const* outs,
                                          const void* const* ins, void* const* ws, const size_t* ws_bytes,
                                          hipStream_t st);
