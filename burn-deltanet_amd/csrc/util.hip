// Small utility kernels: the NaN/Inf guard (the reference's `sanity`,
// src/delta/path.rs:198-207, compiled in by its check-nan/check-inf features).

#include "dn_common.hpp"

namespace dn {
namespace {

template <class T>
__global__ __launch_bounds__(256) void nonfinite_kernel(const T* p, size_t n, int* flag) {
  bool bad = false;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    bad |= !isfinite(ld(p, i));
  // Every writer stores the same value, so the plain store needs no atomic.
  if (bad) *flag = 1;
}

}  // namespace

hipError_t launch_nonfinite_scan(const void* p, size_t n, int dtype, int* flag,
                                 hipStream_t stream) {
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (dtype == DN_BF16)
    hipLaunchKernelGGL(nonfinite_kernel<bf16>, dim3(unsigned(blocks)), dim3(256), 0, stream,
                       static_cast<const bf16*>(p), n, flag);
  else
    hipLaunchKernelGGL(nonfinite_kernel<float>, dim3(unsigned(blocks)), dim3(256), 0, stream,
                       static_cast<const float*>(p), n, flag);
  return hipGetLastError();
}

}  // namespace dn
