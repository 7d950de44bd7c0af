// vec engine of libllhip: RMSNorm, RoPE, SiLU, MUL, ADD, QUANT on the datapath
// types (i16 in, i16/i8 out; NUMERICS.md "RMSNorm", "RoPE", "SiLU",
// "Elementwise"), plus the host-loop helpers embedding gather and argmax
// (golden.py:369-377).
#include "../../include/llhip.h"
#include "common.h"

namespace llhip {

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)v, off);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// ---------------------------------------------------------------------------------------
// RMSNorm (golden.py:124-137): one wave per row
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const int16_t* __restrict__ x, int64_t rows, int K, int64_t ldx,
                                                      const int16_t* __restrict__ g, uint32_t eps_t, uint32_t C, int sh,
                                                      int16_t* __restrict__ y, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int16_t* xr = x + row * ldx;
  uint64_t ss = 0;
  for (int k = lane; k < K; k += 64) {
    const int32_t v = xr[k];
    ss += (uint64_t)(int64_t)(v * v);  // |v| <= 2^15: v*v <= 2^30 fits int32
  }
  ss = wave_sum_u64(ss);
  const uint64_t tt = ss + eps_t;  // < 2^48: the host bounds K so that K * 2^30 + 2^32 < 2^48
  const uint32_t r = isqrt48(tt);
  const uint32_t d = r > 1 ? r : 1u;
  uint32_t inv = C / d;  // C < 2^32, so the quotient already fits u32
  if (inv > 65535u) inv = 65535u;
  int16_t* yr = y + row * ldy;
  for (int k = lane; k < K; k += 64) {
    const int64_t xg = (int64_t)((int32_t)xr[k] * (int32_t)g[k]);
    yr[k] = (int16_t)sat16(rshr(xg * (int64_t)inv, sh));
  }
}

// ---------------------------------------------------------------------------------------
// elementwise
// ---------------------------------------------------------------------------------------
__global__ void quant_kernel(const int16_t* __restrict__ x, int64_t n, int64_t M, int S, int8_t* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (int8_t)sat8(mulshift(x[i], M, S));
}

__global__ void silu_kernel(const int16_t* __restrict__ x, int64_t n, int64_t Mi, int Si, int sh, int16_t* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (int16_t)silu16(x[i], Mi, Si, sh);
}

__global__ void vmul_kernel(const int16_t* __restrict__ a, const int16_t* __restrict__ b, int64_t n, int sh,
                            int16_t* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (int16_t)sat16(rshr((int64_t)((int32_t)a[i] * (int32_t)b[i]), sh));
}

__global__ void vadd_kernel(const int16_t* __restrict__ a, const int16_t* __restrict__ b, int64_t n, int sh,
                            int16_t* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (int16_t)sat16((int64_t)a[i] + rshr(b[i], sh));
}

static unsigned ew_blocks(int64_t n) {
  int64_t b = ceil_div(n, 256);
  if (b > 8192) b = 8192;
  return (unsigned)(b < 1 ? 1 : b);
}

// ---------------------------------------------------------------------------------------
// RoPE (golden.py:141-158): thread per (row, head, i < D/2)
// ---------------------------------------------------------------------------------------
__global__ void rope_kernel(const int16_t* __restrict__ x, int64_t M, int H, int D, int64_t ldx,
                            const int16_t* __restrict__ cos_tab, const int16_t* __restrict__ sin_tab, int pos,
                            const int32_t* __restrict__ pos_dev, int16_t* __restrict__ y, int64_t ldy) {
  const int half = D / 2;
  const int64_t total = M * H * half;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t m = idx / ((int64_t)H * half);
  const int rem = (int)(idx % ((int64_t)H * half));
  const int h = rem / half, i = rem % half;
  const int p0 = pos_dev ? *pos_dev : pos;
  const int64_t trow = (int64_t)(p0 + m) * half;
  const int64_t c = cos_tab[trow + i], s = sin_tab[trow + i];
  const int64_t a = x[m * ldx + h * D + i], b = x[m * ldx + h * D + half + i];
  y[m * ldy + h * D + i] = (int16_t)sat16(rshr(a * c - b * s, 14));
  y[m * ldy + h * D + half + i] = (int16_t)sat16(rshr(b * c + a * s, 14));
}

// ---------------------------------------------------------------------------------------
// embedding gather (golden.py:369-373) and argmax (golden.py:376-377)
// ---------------------------------------------------------------------------------------
__global__ void embed_kernel(const int16_t* __restrict__ embed, int64_t dim, const int32_t* __restrict__ tokens,
                             int64_t n_tokens, int64_t M, int16_t* __restrict__ rows) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * dim) return;
  const int64_t m = idx / dim, d = idx % dim;
  rows[idx] = m < n_tokens ? embed[(int64_t)tokens[m] * dim + d] : (int16_t)0;
}

// key orders by value, then by lower index: larger key = better
__device__ __forceinline__ uint64_t amax_key(int v, int64_t i) {
  return ((uint64_t)(uint32_t)(v + 32768) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

__global__ __launch_bounds__(256) void argmax_kernel(const int16_t* __restrict__ logits, int64_t ld, int64_t vocab,
                                                     int32_t* __restrict__ idx) {
  __shared__ uint64_t best[4];
  const int64_t row = blockIdx.x;
  const int16_t* lr = logits + row * ld;
  uint64_t key = 0;
  for (int64_t i = threadIdx.x; i < vocab; i += 256) {
    const uint64_t k = amax_key(lr[i], i);
    key = k > key ? k : key;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)key, off);
    uint32_t hi = __shfl_xor((uint32_t)(key >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    key = o > key ? o : key;
  }
  if ((threadIdx.x & 63) == 0) best[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t k = best[0];
    for (int w = 1; w < 4; ++w) k = best[w] > k ? best[w] : k;
    idx[row] = (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
  }
}

// Decode-loop step on the device: first argmax of logits[0:vocab] -> *token, the row and the
// token stored in record slot *step, then *pos += 1 and *step += 1.  Blocks reduce their slice
// to a 64-bit key (value, then lowest index) with one atomicMax; the last block to arrive
// publishes the token, advances the state and clears the workspace slots.
__global__ __launch_bounds__(256) void greedy_step_kernel(const int16_t* __restrict__ logits, int64_t vocab,
                                                          int32_t* token, int32_t* pos, int32_t* step,
                                                          int16_t* __restrict__ ring_rows, int64_t ring_ld,
                                                          int32_t* ring_tok, int64_t ring_cap,
                                                          unsigned long long* key_slot, uint32_t* counter) {
  __shared__ uint64_t best[4];
  const int s = *step;
  const bool rec = s < ring_cap;
  int16_t* dst = ring_rows + (int64_t)s * ring_ld;
  uint64_t key = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < vocab; i += stride) {
    const int16_t v = logits[i];
    if (rec) dst[i] = v;
    const uint64_t k = amax_key(v, i);
    key = k > key ? k : key;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)key, off);
    uint32_t hi = __shfl_xor((uint32_t)(key >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    key = o > key ? o : key;
  }
  if ((threadIdx.x & 63) == 0) best[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x != 0) return;
  uint64_t k = best[0];
  for (int w = 1; w < 4; ++w) k = best[w] > k ? best[w] : k;
  atomicMax(key_slot, (unsigned long long)k);
  __threadfence();
  const uint32_t prev = atomicAdd(counter, 1u);
  if (prev != gridDim.x - 1) return;
  __threadfence();
  const unsigned long long win = atomicExch(key_slot, 0ull);
  const int32_t idx = (int32_t)(0xFFFFFFFFu - (uint32_t)(win & 0xFFFFFFFFull));
  *token = idx;
  if (rec) ring_tok[s] = idx;
  *pos = *pos + 1;
  *step = s + 1;
  atomicExch(counter, 0u);
}

}  // namespace llhip

using namespace llhip;

extern "C" {

int llhip_rmsnorm(const int16_t* x, int64_t rows, int64_t K, int64_t ldx, const int16_t* g, int64_t eps_t, int64_t C,
                  int64_t sh_post, int16_t* y, int64_t ldy, void* stream) {
  if (rows < 0 || K < 0) return fail(-EINVAL, "rmsnorm: negative shape");
  if (rows == 0) return 0;
  if (!u32_ok(eps_t) || !u32_ok(C) || !shift_ok(sh_post)) return fail(-EINVAL, "rmsnorm: eps_t/C must be u32, sh_post in [0,63]");
  // isqrt48 domain: sum of K squares of i16 (each <= 2^30) plus eps_t must stay below 2^48
  if (K >= (int64_t)((1ull << 48) - (1ull << 32)) >> 30) return fail(-ERANGE, "isqrt48 input out of range: K=%lld", (long long)K);
  if (ldx < K || ldy < K) return fail(-EINVAL, "rmsnorm: leading dimension too small");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream, x, rows,
                     (int)K, ldx, g, (uint32_t)eps_t, (uint32_t)C, (int)sh_post, y, ldy);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_quant(const int16_t* x, int64_t n, int64_t M, int64_t S, int8_t* y, void* stream) {
  if (!u32_ok(M) || !shift_ok(S)) return fail(-EINVAL, "quant: M must be u32, S in [0,63]");
  if (n <= 0) return n < 0 ? fail(-EINVAL, "quant: negative count") : 0;
  hipLaunchKernelGGL(quant_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t)stream, x, n, M, (int)S, y);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_silu(const int16_t* x, int64_t n, int64_t Mi, int64_t Si, int64_t sh_out, int16_t* y, void* stream) {
  if (!u32_ok(Mi) || !shift_ok(Si) || !shift_ok(sh_out)) return fail(-EINVAL, "silu: Mi must be u32, shifts in [0,63]");
  if (n <= 0) return n < 0 ? fail(-EINVAL, "silu: negative count") : 0;
  hipLaunchKernelGGL(silu_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t)stream, x, n, Mi, (int)Si, (int)sh_out, y);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_vmul(const int16_t* a, const int16_t* b, int64_t n, int64_t sh, int16_t* y, void* stream) {
  if (!shift_ok(sh)) return fail(-EINVAL, "mul: sh out of [0,63]");
  if (n <= 0) return n < 0 ? fail(-EINVAL, "mul: negative count") : 0;
  hipLaunchKernelGGL(vmul_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t)stream, a, b, n, (int)sh, y);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_vadd(const int16_t* a, const int16_t* b, int64_t n, int64_t sh_b, int16_t* y, void* stream) {
  if (!shift_ok(sh_b)) return fail(-EINVAL, "add: sh_b out of [0,63]");
  if (n <= 0) return n < 0 ? fail(-EINVAL, "add: negative count") : 0;
  hipLaunchKernelGGL(vadd_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t)stream, a, b, n, (int)sh_b, y);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_rope(const int16_t* x, int64_t M, int64_t H, int64_t D, int64_t ldx, const int16_t* cos_tab,
               const int16_t* sin_tab, int64_t table_rows, int64_t pos, const int32_t* pos_dev, int16_t* y,
               int64_t ldy, void* stream) {
  if (M < 0 || H < 0 || D < 0 || D % 2) return fail(-EINVAL, "rope: bad geometry (D must be even)");
  if (ldx < H * D || ldy < H * D) return fail(-EINVAL, "rope: leading dimension too small");
  if (!pos_dev && (pos < 0 || pos + M > table_rows)) return fail(-ERANGE, "rope: positions exceed the table");
  const int64_t total = M * H * (D / 2);
  if (total == 0) return 0;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, x, M, (int)H,
                     (int)D, ldx, cos_tab, sin_tab, (int)pos, pos_dev, y, ldy);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_embed_rows(const int16_t* embed, int64_t vocab_rows, int64_t dim, const int32_t* tokens, int64_t n_tokens,
                     int64_t M, int16_t* rows, void* stream) {
  if (n_tokens < 0 || n_tokens > M || dim < 0 || vocab_rows <= 0) return fail(-EINVAL, "embed_rows: bad shape");
  if (M * dim == 0) return 0;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)ceil_div(M * dim, 256)), dim3(256), 0, (hipStream_t)stream, embed, dim,
                     tokens, n_tokens, M, rows);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_greedy_step(const int16_t* logits, int64_t vocab, int32_t* token, int32_t* pos, int32_t* step,
                      int16_t* ring_rows, int64_t ring_ld, int32_t* ring_tokens, int64_t ring_cap, void* ws,
                      void* stream) {
  if (vocab <= 0 || vocab > 0x7FFFFFFF || ring_ld < vocab || ring_cap < 0 || !ws || !token || !pos || !step)
    return fail(-EINVAL, "greedy_step: bad arguments");
  char* w = static_cast<char*>(ws) + WS_GREEDY;
  int64_t blocks = ceil_div(vocab, 256 * 8);
  if (blocks > 120) blocks = 120;
  hipLaunchKernelGGL(greedy_step_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, logits, vocab, token,
                     pos, step, ring_rows, ring_ld, ring_tokens, ring_cap, reinterpret_cast<unsigned long long*>(w),
                     reinterpret_cast<uint32_t*>(w + 8));
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_argmax_i16(const int16_t* logits, int64_t rows, int64_t ld, int64_t vocab, int32_t* idx, void* stream) {
  if (rows < 0 || vocab <= 0 || ld < vocab) return fail(-EINVAL, "argmax: bad shape");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, logits, ld, vocab, idx);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

}  // extern "C"
