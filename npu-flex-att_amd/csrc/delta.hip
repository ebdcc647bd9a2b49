// Backward pre-kernel: Delta[b, h, i] = sum_d O[b,h,i,d] * dO[b,h,i,d] in fp32.
//
// Replaces the torch op of npu_flash_attention.py:681-685.  HBM-bound: each
// row of O and dO is read once with 16-byte loads; 16 lanes share a row and
// reduce with lane shuffles.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

namespace flexatt {

template <class T>
__global__ __launch_bounds__(256) void delta_kernel(DeltaArgs a) {
  constexpr int EPC = 16 / sizeof(T);  // elements per 16-byte chunk
  const int tid = threadIdx.x, ln = tid & 15;
  if (a.zero && blockIdx.x == 0 && tid < 4) a.zero[tid] = 0;  // the next kernels' work queues
  const int64_t row = (int64_t)blockIdx.x * 16 + (tid >> 4);
  const int64_t rows = (int64_t)a.B * a.H * a.S;
  if (row >= rows) return;
  const int s = (int)(row % a.S);
  const int64_t bh = row / a.S;
  const int hh = (int)(bh % a.H), b = (int)(bh / a.H);
  const T* op = (const T*)a.o.data + b * a.o.sb + hh * a.o.sh + (int64_t)s * a.o.ss;
  const T* dp = (const T*)a.dout.data + b * a.dout.sb + hh * a.dout.sh + (int64_t)s * a.dout.ss;
  float sum = 0.f;
  for (int c = ln; c * EPC < a.D; c += 16) {
    const i32x4 x = ld_global16(op + c * EPC), y = ld_global16(dp + c * EPC);
    const T* xe = (const T*)&x;
    const T* ye = (const T*)&y;
#pragma unroll
    for (int e = 0; e < EPC; ++e) sum = fmaf(to_f32<T>(xe[e]), to_f32<T>(ye[e]), sum);
  }
  sum += __shfl_xor(sum, 8);
  sum += __shfl_xor(sum, 4);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 1);
  if (ln == 0) a.delta[row] = sum;
}

hipError_t bwd_delta(int dtype, const DeltaArgs& a, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H * a.S;
  const dim3 grid((unsigned)((rows + 15) / 16)), block(256);
  switch (dtype) {
    case FLEXATT_F32: hipLaunchKernelGGL(delta_kernel<float>, grid, block, 0, st, a); break;
    case FLEXATT_F16: hipLaunchKernelGGL(delta_kernel<_Float16>, grid, block, 0, st, a); break;
    case FLEXATT_BF16: hipLaunchKernelGGL(delta_kernel<__bf16>, grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace flexatt
