// Host-side internal declarations shared by the translation units of libevamx.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace evamx {

void set_error(const char* fmt, ...);

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
