// Raw-row tail of a gated-delta layer, gfx950: the generalisation of the reference's conv history roll
// (HIST_UPDATE, web/public/engine/wgsl.js:420-434). After a call, the rows [state_pos - 3, P + L) are kept so that
// the next call can rebuild the conv history and replay the rows after the stored state position. Only the conv
// channels and the a/b gate columns are copied (z is not needed for replay). The copy reads only the call's input
// rows and the tail it resumed from, never a mixer's output, so one launch serves every gated-delta layer of a call.
#include "ha_kernels.h"

namespace ha {
namespace {

// grid (rows, B, layers). U is the copy unit: the element type, or 16 bytes when every span and row is aligned.
template <typename T, typename U>
__global__ __launch_bounds__(256) void tail_update_kernel(TailArgs a) {
  constexpr int kPer = sizeof(U) / sizeof(T);  // elements per unit
  const int i = blockIdx.x, b = blockIdx.y, ly = blockIdx.z;
  const int r = a.dst_first + i;  // absolute row
  const T* src = r < a.P
      ? static_cast<const T*>(a.tail[ly]) + ((size_t)b * a.tail_cap_in + (r - (a.s0 - (a.KC - 1)))) * a.stride
      : static_cast<const T*>(a.in[ly]) + ((size_t)b * a.L + (r - a.P)) * a.stride;
  T* dst = static_cast<T*>(a.tail_out[ly]) + ((size_t)b * a.tail_cap_out + i) * a.stride;
  const U* s1 = reinterpret_cast<const U*>(src);
  U* d1 = reinterpret_cast<U*>(dst);
  for (int c = threadIdx.x; c < a.C / kPer; c += blockDim.x) d1[c] = s1[c];
  const U* s2 = reinterpret_cast<const U*>(src + a.ab_off);
  U* d2 = reinterpret_cast<U*>(dst + a.ab_off);
  for (int c = threadIdx.x; c < a.ab_n / kPer; c += blockDim.x) d2[c] = s2[c];
}

struct alignas(16) U16 {
  unsigned w[4];
};

template <typename T>
hipError_t launch_typed(const TailArgs& a, int rows, hipStream_t s) {
  constexpr int per = 16 / sizeof(T);
  bool vec = a.C % per == 0 && a.ab_off % per == 0 && a.ab_n % per == 0 && a.stride % per == 0;
  for (int l = 0; l < a.n && vec; l++)
    vec = ((uintptr_t)a.in[l] | (uintptr_t)a.tail[l] | (uintptr_t)a.tail_out[l]) % 16 == 0;
  dim3 grid(rows, a.B, a.n), block(256);
  if (vec)
    hipLaunchKernelGGL((tail_update_kernel<T, U16>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((tail_update_kernel<T, T>), grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_tail_update(const TailArgs& a, hipStream_t s) {
  const int rows = a.P + a.L - a.dst_first;
  if (rows <= 0 || a.n <= 0) return hipSuccess;
  if (rows > a.tail_cap_out || a.n > kTailLayers) return hipErrorInvalidValue;
  return a.dtype == 0 ? launch_typed<float>(a, rows, s) : launch_typed<_Float16>(a, rows, s);
}

}  // namespace ha
