// float-side engine of libllhip: the reductions and rescalings of activation calibration and
// SmoothQuant over fp32 tensors resident on the GPU (python/llaccel/calibrate.py,
// python/llaccel/smoothquant.py).
//
//   llhip_f32_absmax           running max |x| per column and over the tensor (calibrate.py:56-66,
//                              smoothquant.py:95-99); non-negative floats order like their bit
//                              patterns, so the maxima are integer atomic maxima and exact in any
//                              order.  Non-finite values are counted, not folded in.
//   llhip_f32_rms_min          running min over rows of sqrt(mean(x^2)) in double
//                              (calibrate.py:67-72)
//   llhip_f32_rescale          in place x * col_mul[c], then / col_div[c], then / row_div[r], each an
//                              IEEE fp32 operation (smoothquant.py:250-261 applies them one pass at a
//                              time, so the results are the reference's bit for bit)
//   llhip_f32_smooth_objective the weight terms of smoothquant.py:152-163: per row w = W * s, its
//                              int8 grid step max|w| / 127 (at least 1e-30 / 127), q = round-half-even
//                              (w / step) clamped to [-128, 127] times the step, and the sums over
//                              the matrix of w^2 * act_err and (q - w)^2 * act_energy, every product
//                              rounded in fp32 as torch does and summed in double
#include <algorithm>

#include "../../include/llhip.h"
#include "common.h"

#pragma clang fp contract(off)

namespace llhip {

__device__ __forceinline__ bool finite_f32(uint32_t b) { return (b & 0x7F800000u) != 0x7F800000u; }

__device__ __forceinline__ void atomic_max_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block (256 threads) = 256 consecutive columns x a range of rows; grid (column blocks, row blocks).
__global__ __launch_bounds__(256) void f32_absmax_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                         int64_t ld, int64_t rows_per_block, float* col_max,
                                                         float* amax, int32_t* nonfinite) {
  __shared__ uint32_t red[4];
  __shared__ int32_t bad[4];
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block, r1 = std::min<int64_t>(rows, r0 + rows_per_block);
  uint32_t m = 0;
  int32_t nb = 0;
  if (c < cols) {
    for (int64_t r = r0; r < r1; ++r) {
      const uint32_t b = __float_as_uint(x[r * ld + c]) & 0x7FFFFFFFu;
      if (finite_f32(b))
        m = max(m, b);
      else
        ++nb;
    }
    if (col_max && r1 > r0) atomic_max_u32(reinterpret_cast<uint32_t*>(col_max) + c, m);
  }
  // tensor maximum and non-finite count: one atomic per block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int o = 32; o > 0; o >>= 1) {
    m = max(m, (uint32_t)__shfl_xor((int)m, o));
    nb += __shfl_xor(nb, o);
  }
  if (lane == 0) {
    red[wave] = m;
    bad[wave] = nb;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t bm = max(max(red[0], red[1]), max(red[2], red[3]));
    const int32_t bn = bad[0] + bad[1] + bad[2] + bad[3];
    if (amax) atomic_max_u32(reinterpret_cast<uint32_t*>(amax), bm);
    if (bn) atomicAdd(nonfinite, bn);
  }
}

// one wave per row: sum of squares in double (each square of an fp32 value is exact in double)
__global__ __launch_bounds__(256) void f32_rms_min_kernel(const float* __restrict__ x, int64_t rows, int64_t width,
                                                          double* out_min) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * width;
  double s = 0.0;
  for (int64_t i = lane; i < width; i += 64) {
    const double v = xr[i];
    s += v * v;
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) {
    const double rms = sqrt(s / (double)width);
    __hip_atomic_fetch_min(reinterpret_cast<unsigned long long*>(out_min), (unsigned long long)__double_as_longlong(rms),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(256) void f32_rescale_kernel(float* x, int64_t rows, int64_t cols, int64_t ld,
                                                          const float* __restrict__ col_mul,
                                                          const float* __restrict__ col_div,
                                                          const float* __restrict__ row_div) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cols, c = i - r * cols;
    float v = x[r * ld + c];
    if (col_mul) v = v * col_mul[c];
    if (col_div) v = v / col_div[c];
    if (row_div) v = v / row_div[r];
    x[r * ld + c] = v;
  }
}

// one wave per row; the row is read twice (abs-max, then the error terms), the second time from L2
__global__ __launch_bounds__(256) void f32_smooth_objective_kernel(const float* __restrict__ W, int64_t rows,
                                                                   int64_t cols, const float* __restrict__ s,
                                                                   const float* __restrict__ act_err,
                                                                   const float* __restrict__ act_energy, double* out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* wr = W + row * cols;
  float m = 0.0f;
  for (int64_t i = lane; i < cols; i += 64) m = fmaxf(m, fabsf(wr[i] * s[i]));
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  const float step = fmaxf(m, 1e-30f) / 127.0f;
  double e1 = 0.0, e2 = 0.0;
  for (int64_t i = lane; i < cols; i += 64) {
    const float w = wr[i] * s[i];
    const float q = fminf(fmaxf(rintf(w / step), -128.0f), 127.0f) * step;
    const float d = q - w;
    e1 += (double)((w * w) * act_err[i]);
    e2 += (double)((d * d) * act_energy[i]);
  }
  for (int o = 32; o > 0; o >>= 1) {
    e1 += __shfl_xor(e1, o);
    e2 += __shfl_xor(e2, o);
  }
  if (lane == 0) {
    atomicAdd(out, e1);
    atomicAdd(out + 1, e2);
  }
}

unsigned grid_blocks(int64_t n, int64_t per) {
  return (unsigned)std::min<int64_t>(std::max<int64_t>(ceil_div(n, per), 1), 65535);
}

}  // namespace llhip

using namespace llhip;

extern "C" int llhip_f32_absmax(const float* x, int64_t rows, int64_t cols, int64_t ld, float* col_max, float* amax,
                                int32_t* nonfinite, void* stream) {
  if (rows < 0 || cols < 0 || ld < cols) return fail(-EINVAL, "f32_absmax: bad shape");
  if ((rows && cols && !x) || !nonfinite) return fail(-EINVAL, "f32_absmax: null argument");
  if (rows == 0 || cols == 0) return 0;
  // enough row blocks that the grid fills the GPU, at least 16 rows each
  const int64_t cblocks = ceil_div(cols, 256);
  const int64_t want = std::max<int64_t>(1, ceil_div(4 * (int64_t)current_cu_count(), cblocks));
  const int64_t rpb = std::max<int64_t>(16, ceil_div(rows, want));
  const int64_t rblocks = ceil_div(rows, rpb);
  if (cblocks > INT32_MAX || rblocks > 65535) return fail(-EINVAL, "f32_absmax: tensor too large");
  hipLaunchKernelGGL(f32_absmax_kernel, dim3((unsigned)cblocks, (unsigned)rblocks), dim3(256), 0, (hipStream_t)stream, x,
                     rows, cols, ld, rpb, col_max, amax, nonfinite);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_f32_rms_min(const float* x, int64_t rows, int64_t width, double* out_min, void* stream) {
  if (rows < 0 || width <= 0) return fail(-EINVAL, "f32_rms_min: bad shape");
  if ((rows && !x) || !out_min) return fail(-EINVAL, "f32_rms_min: null argument");
  if (rows == 0) return 0;
  if (ceil_div(rows, 4) > INT32_MAX) return fail(-EINVAL, "f32_rms_min: too many rows");
  hipLaunchKernelGGL(f32_rms_min_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream, x, rows,
                     width, out_min);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_f32_rescale(float* x, int64_t rows, int64_t cols, int64_t ld, const float* col_mul,
                                 const float* col_div, const float* row_div, void* stream) {
  if (rows < 0 || cols < 0 || ld < cols) return fail(-EINVAL, "f32_rescale: bad shape");
  if (rows && cols && !x) return fail(-EINVAL, "f32_rescale: null tensor");
  if (rows == 0 || cols == 0) return 0;
  hipLaunchKernelGGL(f32_rescale_kernel, dim3(grid_blocks(rows * cols, 256 * 4)), dim3(256), 0, (hipStream_t)stream, x,
                     rows, cols, ld, col_mul, col_div, row_div);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_f32_smooth_objective(const float* W, int64_t rows, int64_t cols, const float* scales,
                                          const float* act_err, const float* act_energy, double* out, void* stream) {
  if (rows < 0 || cols <= 0) return fail(-EINVAL, "f32_smooth_objective: bad shape");
  if ((rows && !W) || !scales || !act_err || !act_energy || !out)
    return fail(-EINVAL, "f32_smooth_objective: null argument");
  if (rows == 0) return 0;
  if (ceil_div(rows, 4) > INT32_MAX) return fail(-EINVAL, "f32_smooth_objective: too many rows");
  hipLaunchKernelGGL(f32_smooth_objective_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                     W, rows, cols, scales, act_err, act_energy, out);
  LLHIP_LAUNCH_CHECK();
  return 0;
}
