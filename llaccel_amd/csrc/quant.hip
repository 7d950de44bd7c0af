// quantizer engine of libllhip: the float -> integer conversions of the reference quantizer's
// weights (python/llaccel/refquant.py), exact to its float64 arithmetic.
//
//   llhip_quant_rows_i8  per-output-channel int8 weights: s[n] = max|W[n,:]| / 127 (an all-zero
//                        row gets 1), q = llround(clip(W / s[n], -128, 127))   (refquant.py:137-141,
//                        119-125); one workgroup per row, the row's abs-max as an integer max over
//                        the bit patterns of |w| (non-negative floats order like their bits), then
//                        the row re-read (from L2) and converted
//   llhip_quant_i16      i16 tensors at exponent e: llround(clip(x * 2^-e, -32768, 32767))
//                        (refquant.py:128-134)
//
// llround is C's: nearest integer, halves away from zero (refquant.py:61-72).  Every f32 input is
// exactly a double; the division by s and the scaling by 2^-e are IEEE double operations, as in
// numpy, so the results are the reference's bit for bit.  A non-finite input sets *status.
#include <algorithm>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {

__device__ __forceinline__ double llround_away(double x) {
  const double t = trunc(x);
  const double f = x - t;  // exact: |x| < 2^52
  return f >= 0.5 ? t + 1.0 : (f <= -0.5 ? t - 1.0 : t);
}

__device__ __forceinline__ bool finite_bits(uint32_t b) { return (b & 0x7F800000u) != 0x7F800000u; }

constexpr int QT = 256;  // threads per row

template <bool VEC>
__global__ __launch_bounds__(QT) void quant_rows_i8_kernel(const float* __restrict__ w, int64_t K, int64_t ldw,
                                                          int8_t* __restrict__ q, int64_t ldq,
                                                          double* __restrict__ scales, int32_t* status) {
  __shared__ uint32_t red[QT / 64];
  __shared__ int bad[QT / 64];
  const int64_t n = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* row = w + n * ldw;
  int8_t* qrow = q + n * ldq;
  uint32_t amax = 0;
  bool ok = true;
  if (VEC) {
    for (int64_t c = tid; c < K / 4; c += QT) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + 4 * c);
      const uint32_t b[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ok = ok && finite_bits(b[i]);
        amax = max(amax, b[i] & 0x7FFFFFFFu);
      }
    }
  } else {
    for (int64_t k = tid; k < K; k += QT) {
      const uint32_t b = __float_as_uint(row[k]);
      ok = ok && finite_bits(b);
      amax = max(amax, b & 0x7FFFFFFFu);
    }
  }
  amax = (uint32_t)wave_max_i32((int)amax);  // |w| bits < 2^31: signed order is the float order
  const bool wave_ok = __all(ok);
  if (lane == 0) {
    red[wave] = amax;
    bad[wave] = !wave_ok;
  }
  __syncthreads();
  uint32_t m = red[0];
  int nb = bad[0];
#pragma unroll
  for (int i = 1; i < QT / 64; ++i) {
    m = max(m, red[i]);
    nb |= bad[i];
  }
  if (nb) {
    if (tid == 0) atomicOr(status, 1);
    return;
  }
  const double mx = (double)__uint_as_float(m);
  const double s = mx > 0.0 ? mx / 127.0 : 1.0;
  if (tid == 0) scales[n] = s;
  auto cvt = [&](float x) -> int8_t {
    double v = (double)x / s;
    v = v < -128.0 ? -128.0 : (v > 127.0 ? 127.0 : v);
    return (int8_t)(int)llround_away(v);
  };
  if (VEC) {
    for (int64_t c = tid; c < K / 4; c += QT) {
      const float4 v = *reinterpret_cast<const float4*>(row + 4 * c);
      const uint32_t p = (uint32_t)(uint8_t)cvt(v.x) | ((uint32_t)(uint8_t)cvt(v.y) << 8) |
                         ((uint32_t)(uint8_t)cvt(v.z) << 16) | ((uint32_t)(uint8_t)cvt(v.w) << 24);
      *reinterpret_cast<uint32_t*>(qrow + 4 * c) = p;
    }
  } else {
    for (int64_t k = tid; k < K; k += QT) qrow[k] = cvt(row[k]);
  }
}

__global__ void quant_i16_kernel(const float* __restrict__ x, int64_t n, int e, int16_t* __restrict__ y,
                                 int32_t* status) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float f = x[i];
    if (!finite_bits(__float_as_uint(f))) {
      atomicOr(status, 1);
      y[i] = 0;
      continue;
    }
    double v = ldexp((double)f, -e);
    v = v < -32768.0 ? -32768.0 : (v > 32767.0 ? 32767.0 : v);
    y[i] = (int16_t)(int)llround_away(v);
  }
}

}  // namespace llhip

using namespace llhip;

extern "C" int llhip_quant_rows_i8(const float* w, int64_t N, int64_t K, int64_t ldw, int8_t* q, int64_t ldq,
                                   double* scales, int32_t* status, void* stream) {
  if (N < 0 || K < 0 || ldw < K || ldq < K) return fail(-EINVAL, "quant_rows_i8: bad shape");
  if (N > INT32_MAX) return fail(-EINVAL, "quant_rows_i8: too many rows");
  if (N == 0) return 0;
  if (!w || !q || !scales || !status) return fail(-EINVAL, "quant_rows_i8: null operand");
  const bool vec = K % 4 == 0 && ldw % 4 == 0 && ldq % 4 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)q % 4 == 0;
  if (vec)
    hipLaunchKernelGGL(quant_rows_i8_kernel<true>, dim3((unsigned)N), dim3(QT), 0, (hipStream_t)stream, w, K, ldw, q,
                       ldq, scales, status);
  else
    hipLaunchKernelGGL(quant_rows_i8_kernel<false>, dim3((unsigned)N), dim3(QT), 0, (hipStream_t)stream, w, K, ldw, q,
                       ldq, scales, status);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_quant_i16(const float* x, int64_t n, int64_t e, int16_t* y, int32_t* status, void* stream) {
  if (n < 0) return fail(-EINVAL, "quant_i16: bad size");
  if (e < -1074 || e > 1074) return fail(-EINVAL, "quant_i16: exponent out of range");
  if (n == 0) return 0;
  if (!x || !y || !status) return fail(-EINVAL, "quant_i16: null operand");
  const int blocks = (int)std::min<int64_t>(ceil_div(n, 256), 8 * current_cu_count());
  hipLaunchKernelGGL(quant_i16_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x, n, (int)e, y,
                     status);
  LLHIP_LAUNCH_CHECK();
  return 0;
}
