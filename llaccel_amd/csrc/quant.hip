// quantizer engine of libllhip: the float -> integer conversions of the reference quantizer's
// weights (python/llaccel/refquant.py), exact to its float64 arithmetic.
//
//   llhip_quant_rows_i8  per-output-channel int8 weights: s[n] = max|W[n,:]| / 127 (an all-zero
//                        row gets 1), q = llround(clip(W / s[n], -128, 127))   (refquant.py:137-141,
//                        119-125); the row's abs-max is an integer max over the bit patterns of |w|
//                        (non-negative floats order like their bits).  Rows of up to 4096 aligned
//                        floats: one wave per row held in registers; longer or unaligned rows: one
//                        workgroup per row, read twice (the second time from L2)
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

// One wave per row, the row in registers (CH 16-byte chunks per lane, K <= 256 * CH, K % 4 == 0):
// the abs-max is a wave reduction, the conversion reads the registers again -- no LDS, no barrier,
// every row read once; each wave's next row is loaded while this one is converted.
//
// The conversion needs only the integer that w / s rounds to.  It is taken from the float32
// product w * (1/s) (relative error below 3 * 2^-24, so within 2^-15 of the exact quotient, whose
// magnitude is at most 127 + 2^-40); only a product within 2^-12 of a half-integer is settled by
// the exact float64 division.  llround(clip(q, -128, 127)) equals the rounded q clamped to
// [-128, 127], so the clip is applied to the integer.
// Rows whose abs-max is below 2^-100 (1/s would leave the float32 range) take the float64 path for
// every element; in the others a float32 subnormal quotient is far below 0.5 either way.
__device__ __forceinline__ int32_t quant_one(uint32_t bits, float r32, double s, bool fast) {
  const float x = __uint_as_float(bits);
  const float qa = x * r32;
  const float t = truncf(qa);
  const float f = qa - t;  // exact: |qa| < 2^23
  int32_t v;
  if (!fast || fabsf(fabsf(f) - 0.5f) < 0.000244140625f) {  // 2^-12: settle the tie in float64
    v = (int32_t)llround_away((double)x / s);
  } else {
    v = (int32_t)t + (f > 0.5f ? 1 : 0) - (f < -0.5f ? 1 : 0);
  }
  return v < -128 ? -128 : (v > 127 ? 127 : v);
}

template <int CH>
__device__ __forceinline__ void load_row(const float* row, int lane, int kc, uint4 (&v)[CH]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int i = lane + 64 * c;
    v[c] = i < kc ? *reinterpret_cast<const uint4*>(row + 4 * i) : make_uint4(0u, 0u, 0u, 0u);
  }
}

template <int CH>
__global__ __launch_bounds__(256) void quant_rows_i8_wave(const float* __restrict__ w, int64_t N, int64_t K,
                                                          int64_t ldw, int8_t* __restrict__ q, int64_t ldq,
                                                          double* __restrict__ scales, int32_t* status) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int kc = (int)(K >> 2);  // 16-byte chunks per row
  int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  uint4 v[CH];
  if (n < N) load_row<CH>(w + n * ldw, lane, kc, v);
  for (; n < N; n += nw) {
    uint4 nx[CH];
    if (n + nw < N) load_row<CH>(w + (n + nw) * ldw, lane, kc, nx);
    uint32_t amax = 0;
    bool ok = true;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t b[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ok = ok && finite_bits(b[j]);
        amax = max(amax, b[j] & 0x7FFFFFFFu);
      }
    }
    amax = (uint32_t)wave_max_i32((int)amax);
    if (__all(ok)) {
      const double mx = (double)__uint_as_float(amax);
      const double s = mx > 0.0 ? mx / 127.0 : 1.0;
      const bool fast = mx >= 0x1p-100;
      const float r32 = fast ? (float)(1.0 / s) : 0.0f;
      if (lane == 0) scales[n] = s;
      int8_t* qrow = q + n * ldq;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int i = lane + 64 * c;
        if (i >= kc) break;
        const uint32_t b[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
        uint32_t pk = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) pk |= (uint32_t)(uint8_t)(int8_t)quant_one(b[j], r32, s, fast) << (8 * j);
        *reinterpret_cast<uint32_t*>(qrow + 4 * i) = pk;
      }
    } else if (lane == 0) {
      atomicOr(status, 1);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) v[c] = nx[c];
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
  if (vec && K <= 256 * 16) {
    // a wave per row: enough waves for every CU to keep 32 rows' loads in flight
    const int blocks = (int)std::min<int64_t>(ceil_div(N, 4), 8 * current_cu_count());
    const hipStream_t s = (hipStream_t)stream;
#define LLHIP_QW(CH) \
  hipLaunchKernelGGL(quant_rows_i8_wave<CH>, dim3((unsigned)blocks), dim3(256), 0, s, w, N, K, ldw, q, ldq, scales, status)
    if (K <= 256)
      LLHIP_QW(1);
    else if (K <= 512)
      LLHIP_QW(2);
    else if (K <= 1024)
      LLHIP_QW(4);
    else if (K <= 2048)
      LLHIP_QW(8);
    else
      LLHIP_QW(16);
#undef LLHIP_QW
    LLHIP_LAUNCH_CHECK();
    return 0;
  }
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
