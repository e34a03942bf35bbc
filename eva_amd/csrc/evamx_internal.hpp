// Host-side internal declarations shared by the translation units of libevamx.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/evamx.h"

namespace evamx {

void set_error(const char* fmt, ...);

// The MoE forward of evamx_moe_forward on a given workspace (validation included); `who` names
// the entry point in error messages. Used by the entry points with a caller's workspace and with
// the library's fixed device scratch; side_stream_ok lets calls of more than 16 tokens run their
// MFMA stages' two kernels concurrently on a side stream (the fixed-scratch entry point creates none).
int moe_forward_ws(const evamx_moe_args* a, void* workspace, size_t workspace_bytes, hipStream_t stream,
                   const char* who, bool side_stream_ok);
size_t moe_workspace_bytes_of(const evamx_moe_shape* shape);
int moe_flags_offset(const evamx_moe_shape* shape, size_t* off);
// n ints at p set to v by a kernel on `stream` (capture-safe, unlike a memset node)
void launch_fill_i32(int* p, int n, int v, hipStream_t stream);
// EVAMX_OK, or EVAMX_ELAUNCH with the message set if the last launch failed
int launched(const char* what);

int launch_dequant(const void* trellis, int in, int out, int k2, void* w, bool scalar, hipStream_t stream);

}  // namespace evamx

namespace evamx {

size_t linear_workspace(int rows, int in, int out, size_t* off_part, size_t* off_sum);
int launch_linear(const void* x, int rows, int in, int out, const void* trellis, const void* suh,
                  const void* svh, int k2, void* y, void* ws, hipStream_t stream);

}  // namespace evamx

namespace evamx {

int launch_bench_decode(int k2, int blocks, int iters, float* sink, hipStream_t stream);
void launch_bench_read(const void* base, int ncg, int rows, int n_waves, float* sink, hipStream_t stream);

}  // namespace evamx
