// reduce_group_f32.hip -- the f32 instantiation of the reduction group launcher.
#include "reduce_group_impl.hpp"

template int mx::run_reduce_group<MX_FLOAT32>(const Desc& d, int n, const int* ops, void* const* outs,
                                          const void* const* ins, void* const* ws, const size_t* ws_bytes,
                                          hipStream_t st);
