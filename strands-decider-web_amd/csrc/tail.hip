// Raw-row tail of a gated-delta layer, gfx950: the generalisation of the reference's conv history roll
// (HIST_UPDATE, web/public/engine/wgsl.js:420-434). After a call, the rows [state_pos - 3, P + L) are kept so that
// the next call can rebuild the conv history and replay the rows after the stored state position. Only the conv
// channels and the a/b gate columns are copied (z is not needed for replay).
#include "ha_kernels.h"

namespace ha {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void tail_update_kernel(TailArgs a) {
  const int i = blockIdx.x, b = blockIdx.y;
  const int r = a.dst_first + i;  // absolute row
  const T* src = r < a.P
      ? static_cast<const T*>(a.tail) + ((size_t)b * a.tail_cap_in + (r - (a.s0 - (a.KC - 1)))) * a.stride
      : static_cast<const T*>(a.in) + ((size_t)b * a.L + (r - a.P)) * a.stride;
  T* dst = static_cast<T*>(a.tail_out) + ((size_t)b * a.tail_cap_out + i) * a.stride;
  for (int c = threadIdx.x; c < a.C; c += blockDim.x) dst[c] = src[c];
  for (int c = threadIdx.x; c < a.ab_n; c += blockDim.x) dst[a.ab_off + c] = src[a.ab_off + c];
}

}  // namespace

hipError_t launch_tail_update(const TailArgs& a, hipStream_t s) {
  const int rows = a.P + a.L - a.dst_first;
  if (rows <= 0) return hipSuccess;
  if (rows > a.tail_cap_out) return hipErrorInvalidValue;
  dim3 grid(rows, a.B), block(256);
  if (a.dtype == 0)
    hipLaunchKernelGGL(tail_update_kernel<float>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(tail_update_kernel<_Float16>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace ha
