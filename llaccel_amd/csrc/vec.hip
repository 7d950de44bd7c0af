// vec engine of libllhip: RMSNorm, RoPE, SiLU, MUL, ADD, QUANT on the datapath
// types (i16 in, i16/i8 out; NUMERICS.md "RMSNorm", "RoPE", "SiLU",
// "Elementwise"), plus the host-loop helpers embedding gather and argmax
// (golden.py:369-377).
#include <algorithm>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {

// ---------------------------------------------------------------------------------------
// RMSNorm (golden.py:124-137): one wave per row.  Rows whose K and stride are multiples of 8
// move 16 bytes (8 values) per lane per load, four loads in flight.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const int16_t* __restrict__ x, int64_t rows, int K, int64_t ldx,
                                                      const int16_t* __restrict__ g, uint32_t eps_t, uint32_t C, int sh,
                                                      int16_t* __restrict__ y, int64_t ldy, int vec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int16_t* xr = x + row * ldx;
  int16_t* yr = y + row * ldy;
  uint64_t ss = 0;
  if (vec) {
    const int nch = K >> 3;
    const v4i* xv = reinterpret_cast<const v4i*>(xr);
    for (int c0 = lane; c0 < nch; c0 += 256) {
      v4i b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = c0 + 64 * u < nch ? xv[c0 + 64 * u] : v4i{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int32_t a = lo16(b[u][j]), c = hi16(b[u][j]);
          ss += (uint64_t)(uint32_t)(a * a) + (uint64_t)(uint32_t)(c * c);
        }
    }
    ss = wave_sum_u64(ss);
    const uint32_t inv = rms_inv(ss, eps_t, C);
    const v4i* gv = reinterpret_cast<const v4i*>(g);
    v4i* yv = reinterpret_cast<v4i*>(yr);
    for (int c0 = lane; c0 < nch; c0 += 256) {
      v4i b[4], gg[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool ok = c0 + 64 * u < nch;
        b[u] = ok ? xv[c0 + 64 * u] : v4i{0, 0, 0, 0};
        gg[u] = ok ? gv[c0 + 64 * u] : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (c0 + 64 * u >= nch) break;
        v4i o;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = pack16(rms_apply(lo16(b[u][j]), lo16(gg[u][j]), inv, sh), rms_apply(hi16(b[u][j]), hi16(gg[u][j]), inv, sh));
        yv[c0 + 64 * u] = o;
      }
    }
    return;
  }
  for (int k = lane; k < K; k += 64) {
    const int32_t v = xr[k];
    ss += (uint64_t)(uint32_t)(v * v);
  }
  ss = wave_sum_u64(ss);
  const uint32_t inv = rms_inv(ss, eps_t, C);
  for (int k = lane; k < K; k += 64) yr[k] = rms_apply(xr[k], g[k], inv, sh);
}

// ---------------------------------------------------------------------------------------
// elementwise: 8 consecutive values per thread, 16-byte accesses when aligned
// ---------------------------------------------------------------------------------------
struct EwArgs {
  const int16_t* a;
  const int16_t* b;
  void* y;
  int64_t n;
  int64_t M;  // multiplier (quant M / silu Mi)
  int s0, s1; // shifts
  int aligned;
};

template <int OP>  // 0 quant, 1 silu, 2 vmul, 3 vadd
__device__ __forceinline__ int64_t ew_one(const EwArgs& p, int64_t a, int64_t b) {
  if (OP == 0) return sat8(mulshift(a, p.M, p.s0));
  if (OP == 1) return silu16(a, p.M, p.s0, p.s1);
  if (OP == 2) return sat16(rshr(a * b, p.s0));
  return sat16(a + rshr(b, p.s0));
}

template <int OP>
__global__ __launch_bounds__(256) void ew_kernel(EwArgs p) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i0 >= p.n) return;
  if (p.aligned && i0 + 8 <= p.n) {
    const v4i av = *reinterpret_cast<const v4i*>(p.a + i0);
    v4i bv = {0, 0, 0, 0};
    if (OP >= 2) bv = *reinterpret_cast<const v4i*>(p.b + i0);
    int64_t r[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r[2 * j] = ew_one<OP>(p, lo16(av[j]), lo16(bv[j]));
      r[2 * j + 1] = ew_one<OP>(p, hi16(av[j]), hi16(bv[j]));
    }
    if (OP == 0) {
      int2 o;
      o.x = (int)((uint32_t)(uint8_t)r[0] | (uint32_t)(uint8_t)r[1] << 8 | (uint32_t)(uint8_t)r[2] << 16 |
                  (uint32_t)(uint8_t)r[3] << 24);
      o.y = (int)((uint32_t)(uint8_t)r[4] | (uint32_t)(uint8_t)r[5] << 8 | (uint32_t)(uint8_t)r[6] << 16 |
                  (uint32_t)(uint8_t)r[7] << 24);
      *reinterpret_cast<int2*>(static_cast<int8_t*>(p.y) + i0) = o;
    } else {
      v4i o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack16(r[2 * j], r[2 * j + 1]);
      *reinterpret_cast<v4i*>(static_cast<int16_t*>(p.y) + i0) = o;
    }
    return;
  }
  for (int64_t i = i0; i < p.n && i < i0 + 8; ++i) {
    const int64_t r = ew_one<OP>(p, p.a[i], OP >= 2 ? p.b[i] : 0);
    if (OP == 0)
      static_cast<int8_t*>(p.y)[i] = (int8_t)r;
    else
      static_cast<int16_t*>(p.y)[i] = (int16_t)r;
  }
}

template <int OP>
static int launch_ew(EwArgs p, hipStream_t stream) {
  if (p.n <= 0) return p.n < 0 ? fail(-EINVAL, "negative element count") : 0;
  p.aligned = ((uintptr_t)p.a % 16 == 0) && (!p.b || (uintptr_t)p.b % 16 == 0) && ((uintptr_t)p.y % 16 == 0);
  const int64_t threads = ceil_div(p.n, 8);
  hipLaunchKernelGGL(ew_kernel<OP>, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
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
                            const int16_t* __restrict__ cos_tab, const int16_t* __restrict__ sin_tab,
                            int64_t table_rows, int pos, const int32_t* __restrict__ pos_dev,
                            const int32_t* __restrict__ row_pos, int16_t* __restrict__ y, int64_t ldy) {
  const int half = D / 2;
  const int64_t total = M * H * half;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t m = idx / ((int64_t)H * half);
  const int rem = (int)(idx % ((int64_t)H * half));
  const int h = rem / half, i = rem % half;
  const int64_t pm = row_pos ? (int64_t)row_pos[m] : (int64_t)(pos_dev ? *pos_dev : pos) + m;
  if (pm < 0 || pm >= table_rows) return;  // device positions are checked by the caller; never read past the table
  const int64_t trow = pm * half;
  const int64_t c = cos_tab[trow + i], s = sin_tab[trow + i];
  const int64_t a = x[m * ldx + h * D + i], b = x[m * ldx + h * D + half + i];
  y[m * ldy + h * D + i] = (int16_t)sat16(rshr(a * c - b * s, 14));
  y[m * ldy + h * D + half + i] = (int16_t)sat16(rshr(b * c + a * s, 14));
}

struct RopeJob {
  const int16_t* x;
  int64_t M, ldx, table_rows, qM, ldv, max_seq, slot_stride, total;
  int64_t seq_rows;  // > 0: row m at pos + m % seq_rows in cache slot m / seq_rows
  int H, D, pos, qS;
  const int16_t* cos_tab;
  const int16_t* sin_tab;
  const int32_t* pos_dev;
  const int32_t* row_pos;
  int16_t* y;
  int8_t* yq;
  int8_t* kc;
  const int8_t* v;
  int8_t* vc;
};

// IDX: the index type of the launch (32-bit division where the total allows it)
template <class IDX>
__device__ __forceinline__ void rope_quant_one(const RopeJob& j, IDX idx) {
  const int half = j.D / 2;
  const IDX hh = (IDX)j.H * (IDX)half;
  const int64_t m = (int64_t)(idx / hh);
  const int rem = (int)(idx % hh);
  const int h = rem / half, i = rem % half;
  const int64_t pm = j.row_pos    ? (int64_t)j.row_pos[m]
                     : j.seq_rows ? (int64_t)j.pos + m % j.seq_rows
                                  : (int64_t)(j.pos_dev ? *j.pos_dev : j.pos) + m;
  if (pm < 0 || pm >= j.table_rows) return;  // device positions are checked by the caller; never read past the table
  const int64_t trow = pm * half;
  // i16 operands: the rotation's sums in 64-bit (b c + a s reaches 2^31 when all four are -32768),
  // and the quant of an i16 is exact in double
  const int32_t c = j.cos_tab[trow + i], s = j.sin_tab[trow + i];
  const int64_t o = m * (int64_t)j.H * j.D + (int64_t)h * j.D;
  const int32_t a = j.x[m * j.ldx + h * j.D + i], b = j.x[m * j.ldx + h * j.D + half + i];
  const int16_t y1 = (int16_t)sat16(rshr((int64_t)a * c - (int64_t)b * s, 14));
  const int16_t y2 = (int16_t)sat16(rshr((int64_t)b * c + (int64_t)a * s, 14));
  j.y[o + i] = y1;
  j.y[o + half + i] = y2;
  const double sq = mulshift_scale(j.qM, j.qS);
  const int8_t q1 = (int8_t)mulshift_small_sat(y1, sq, -128.0, 127.0);
  const int8_t q2 = (int8_t)mulshift_small_sat(y2, sq, -128.0, 127.0);
  j.yq[o + i] = q1;
  j.yq[o + half + i] = q2;
  if (j.kc && pm < j.max_seq) {  // never write past a cache
    const int64_t slot = j.row_pos ? m * j.slot_stride : (j.seq_rows ? m / j.seq_rows * j.slot_stride : 0);
    const int64_t dst = slot + ((int64_t)h * j.max_seq + pm) * j.D;
    j.kc[dst + i] = q1;
    j.kc[dst + half + i] = q2;
    if (j.vc) {
      j.vc[dst + i] = j.v[m * j.ldv + (int64_t)h * j.D + i];
      j.vc[dst + half + i] = j.v[m * j.ldv + (int64_t)h * j.D + half + i];
    }
  }
}

// RoPE then quant of the rotated rows in one pass (golden.py:141-158, 119-120); for key rows also
// the layer's kv_write (golden.py:344-351): the quantised keys and the v rows into the caches at
// their positions.  Thread per (row, head, i < D/2) of job a, then of job b (b.total = 0: none).
template <class IDX>
__global__ void rope_quant_kernel(RopeJob a, RopeJob b) {
  const IDX idx = (IDX)blockIdx.x * (IDX)blockDim.x + (IDX)threadIdx.x;
  if (idx < (IDX)a.total)
    rope_quant_one<IDX>(a, idx);
  else if (idx < (IDX)(a.total + b.total))
    rope_quant_one<IDX>(b, idx - (IDX)a.total);
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

__global__ __launch_bounds__(256) void argmax_kernel(const int16_t* __restrict__ logits, int64_t ld, int64_t vocab,
                                                     int32_t* __restrict__ idx) {
  __shared__ uint64_t best[4];
  const int64_t row = blockIdx.x;
  const int16_t* lr = logits + row * ld;
  uint64_t key = 0;
  if ((reinterpret_cast<uintptr_t>(lr) & 15) == 0 && vocab < (1ll << 31) / 2) {
    // 16-byte chunks of 8 values, eight chunks per thread in flight per pass (a pass of one load
    // at a time waits a memory round trip per value)
    const int64_t chunks = vocab / 8;  // whole chunks; the vocab % 8 values after them one at a time
    const Rsrc rr = rsrc(lr, chunks * 16);
    for (int64_t c0 = threadIdx.x; c0 < chunks; c0 += 256 * 8) {
      v4i w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t c = c0 + 256 * u;
        w[u] = ld16(rr, c < chunks ? (uint32_t)(16 * c) : LD_OOB);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t c = c0 + 256 * u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t i = 8 * c + e;
          const int16_t v = (int16_t)((uint32_t)w[u][e >> 1] >> (16 * (e & 1)));
          const uint64_t k = c < chunks ? amax_key(v, i) : 0;
          key = k > key ? k : key;
        }
      }
    }
    if (threadIdx.x < vocab - 8 * chunks) {
      const int64_t i = 8 * chunks + threadIdx.x;
      const uint64_t k = amax_key(lr[i], i);
      key = k > key ? k : key;
    }
  } else {
    for (int64_t i = threadIdx.x; i < vocab; i += 256) {
      const uint64_t k = amax_key(lr[i], i);
      key = k > key ? k : key;
    }
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

// Batch decode step on the device: one workgroup per row (sequence).  Each thread scans 8-element
// chunks keeping its first maximum (strictly greater replaces), then the workgroup keeps the
// largest value and, among equal values, the lowest index -- the first argmax of golden.py:376-377.
constexpr int GR_THREADS = 1024;

__device__ __forceinline__ void block_argmax(int32_t& v, int32_t& i, int32_t* sv, int32_t* si) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int32_t wv = wave_max_i32(v);
  const int32_t wi = -wave_max_i32(v == wv ? -i : INT32_MIN + 1);  // lowest index holding the maximum
  if (lane == 0) {
    sv[wave] = wv;
    si[wave] = wi;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  for (int w = 1; w < nw; ++w)
    if (sv[w] > v || (sv[w] == v && si[w] < i)) {
      v = sv[w];
      i = si[w];
    }
}

__global__ __launch_bounds__(GR_THREADS) void greedy_rows_kernel(const int16_t* __restrict__ logits, int64_t ld,
                                                                 int64_t vocab, int32_t* tokens, int32_t* positions,
                                                                 const int32_t* __restrict__ base,
                                                                 int16_t* __restrict__ ring_rows, int64_t ring_ld,
                                                                 int32_t* ring_tok, int64_t ring_cap, int64_t rows) {
  __shared__ int32_t sv[GR_THREADS / 64], si[GR_THREADS / 64];
  const int r = blockIdx.x;
  const int64_t s = (int64_t)positions[r] - base[r];
  const bool rec = s >= 0 && s < ring_cap;
  const int16_t* lr = logits + (int64_t)r * ld;
  int16_t* dst = ring_rows + (s * rows + r) * ring_ld;
  const Rsrc lrs = rsrc(lr, (vocab + 1) / 2 * 4);  // whole dwords: the range check is per dword
  int32_t best = INT32_MIN, bi = 0;
  // 16-byte chunks of 8 values, GR_PASS chunks per thread in flight per pass (one load at a time
  // waited a memory round trip per chunk: 14 us for 16 rows of 151936), each thread's chunks in
  // ascending order so a strict > keeps the lowest index of its maximum
  constexpr int GR_PASS = 8;
  const int64_t nch = (vocab + 7) / 8;
  for (int64_t c0 = threadIdx.x; c0 < nch; c0 += (int64_t)GR_THREADS * GR_PASS) {
    v4i w[GR_PASS];
#pragma unroll
    for (int u = 0; u < GR_PASS; ++u) {
      const int64_t c = c0 + (int64_t)GR_THREADS * u;
      w[u] = ld16(lrs, c < nch ? (uint32_t)(c * 16) : LD_OOB);  // elements past vocab read zero, skipped
    }
#pragma unroll
    for (int u = 0; u < GR_PASS; ++u) {
      const int64_t c = c0 + (int64_t)GR_THREADS * u;
      if (c >= nch) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t i = c * 8 + e;
        const int32_t v = (e & 1) ? hi16(w[u][e >> 1]) : lo16(w[u][e >> 1]);
        if (i < vocab && v > best) {
          best = v;
          bi = (int32_t)i;
        }
      }
      if (rec) {
        if (c * 8 + 8 <= vocab && ring_ld % 8 == 0) {
          *reinterpret_cast<v4i*>(dst + c * 8) = w[u];
        } else {
          for (int e = 0; e < 8 && c * 8 + e < vocab; ++e)
            dst[c * 8 + e] = (int16_t)((e & 1) ? hi16(w[u][e >> 1]) : lo16(w[u][e >> 1]));
        }
      }
    }
  }
  block_argmax(best, bi, sv, si);
  if (threadIdx.x != 0) return;
  tokens[r] = bi;
  if (rec) ring_tok[s * rows + r] = bi;
  positions[r] = positions[r] + 1;
}


// ---------------------------------------------------------------------------------------
// record verification on the device (long runs checked without downloading every logits row)
// ---------------------------------------------------------------------------------------
// first mismatching element of two i16 row sets: smallest flat index r * cols + c, -1 if none.
// Three stream-ordered launches (set, compare with atomicMin, finish): no memset, so they can be
// captured in a graph.
__global__ void mismatch_init_kernel(unsigned long long* out) { *out = ~0ull; }

__global__ __launch_bounds__(256) void mismatch_kernel(const int16_t* __restrict__ a, int64_t lda,
                                                       const int16_t* __restrict__ b, int64_t ldb, int64_t rows,
                                                       int64_t cols, unsigned long long* out) {
  const int64_t n = rows * cols;
  unsigned long long first = ~0ull;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, c = i % cols;
    if (a[r * lda + c] != b[r * ldb + c]) {
      first = (unsigned long long)i;
      break;  // later indices of this thread are larger
    }
  }
  // wave minimum, then one atomic per wave
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)first, off), hi = __shfl_xor((uint32_t)(first >> 32), off);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    first = o < first ? o : first;
  }
  if ((threadIdx.x & 63) == 0 && first != ~0ull) atomicMin(out, first);
}

__global__ void mismatch_finish_kernel(unsigned long long* out) {
  if (*out == ~0ull) *reinterpret_cast<int64_t*>(out) = -1;
}

// sum over the wave modulo 2^64 (any 64-bit lane values)
__device__ __forceinline__ uint64_t wave_sum_u64_full(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off), hi = __shfl_xor((uint32_t)(v >> 32), off);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// per-row checksum sum_c (c + 1) * (uint16)x[r][c] modulo 2^64: exact, order-independent, and
// position-weighted (a swap of two unequal values changes it); one workgroup per row
__global__ __launch_bounds__(256) void row_checksum_kernel(const int16_t* __restrict__ x, int64_t ld, int64_t cols,
                                                           uint64_t* __restrict__ out) {
  __shared__ uint64_t part[4];
  const int64_t r = blockIdx.x;
  uint64_t acc = 0;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x)
    acc += (uint64_t)(c + 1) * (uint64_t)(uint16_t)x[r * ld + c];
  acc = wave_sum_u64_full(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[r] = part[0] + part[1] + part[2] + part[3];
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
  const int vec = (K % 8 == 0) && (ldx % 8 == 0) && (ldy % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                  ((uintptr_t)y % 16 == 0) && ((uintptr_t)g % 16 == 0);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream, x, rows,
                     (int)K, ldx, g, (uint32_t)eps_t, (uint32_t)C, (int)sh_post, y, ldy, vec);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_quant(const int16_t* x, int64_t n, int64_t M, int64_t S, int8_t* y, void* stream) {
  if (!u32_ok(M) || !shift_ok(S)) return fail(-EINVAL, "quant: M must be u32, S in [0,63]");
  return launch_ew<0>(EwArgs{x, nullptr, y, n, M, (int)S, 0, 0}, (hipStream_t)stream);
}

int llhip_silu(const int16_t* x, int64_t n, int64_t Mi, int64_t Si, int64_t sh_out, int16_t* y, void* stream) {
  if (!u32_ok(Mi) || !shift_ok(Si) || !shift_ok(sh_out)) return fail(-EINVAL, "silu: Mi must be u32, shifts in [0,63]");
  return launch_ew<1>(EwArgs{x, nullptr, y, n, Mi, (int)Si, (int)sh_out, 0}, (hipStream_t)stream);
}

int llhip_vmul(const int16_t* a, const int16_t* b, int64_t n, int64_t sh, int16_t* y, void* stream) {
  if (!shift_ok(sh)) return fail(-EINVAL, "mul: sh out of [0,63]");
  return launch_ew<2>(EwArgs{a, b, y, n, 0, (int)sh, 0, 0}, (hipStream_t)stream);
}

int llhip_vadd(const int16_t* a, const int16_t* b, int64_t n, int64_t sh_b, int16_t* y, void* stream) {
  if (!shift_ok(sh_b)) return fail(-EINVAL, "add: sh_b out of [0,63]");
  return launch_ew<3>(EwArgs{a, b, y, n, 0, (int)sh_b, 0, 0}, (hipStream_t)stream);
}

int llhip_rope(const int16_t* x, int64_t M, int64_t H, int64_t D, int64_t ldx, const int16_t* cos_tab,
               const int16_t* sin_tab, int64_t table_rows, int64_t pos, const int32_t* pos_dev,
               const int32_t* row_pos, int16_t* y, int64_t ldy, void* stream) {
  if (M < 0 || H < 0 || D < 0 || D % 2) return fail(-EINVAL, "rope: bad geometry (D must be even)");
  if (ldx < H * D || ldy < H * D) return fail(-EINVAL, "rope: leading dimension too small");
  if (!pos_dev && !row_pos && (pos < 0 || pos + M > table_rows)) return fail(-ERANGE, "rope: positions exceed the table");
  const int64_t total = M * H * (D / 2);
  if (total == 0) return 0;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, x, M, (int)H,
                     (int)D, ldx, cos_tab, sin_tab, table_rows, (int)pos, pos_dev, row_pos, y, ldy);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

}  // extern "C"

namespace llhip {
// the checks of llhip_rope_quant, and its launch arguments
static int rope_job(const llhip_rope_quant_desc& d, RopeJob& j) {
  const int64_t M = d.M, H = d.H, D = d.D;
  if (M < 0 || H < 0 || D < 0 || D % 2) return fail(-EINVAL, "rope_quant: bad geometry (D must be even)");
  if (d.ldx < H * D) return fail(-EINVAL, "rope_quant: leading dimension too small");
  if (!u32_ok(d.qM) || !shift_ok(d.qS)) return fail(-EINVAL, "rope_quant: quant multiplier must be u32, shift in [0,63]");
  if (d.seq_rows < 0 || (d.seq_rows > 0 && (d.pos_dev || d.row_pos || M % d.seq_rows)))
    return fail(-EINVAL, "rope_quant: sequences of seq_rows rows need M %% seq_rows == 0 and no row positions");
  const int64_t span = d.seq_rows > 0 ? d.seq_rows : M;  // consecutive positions of one sequence
  if (!d.pos_dev && !d.row_pos && (d.pos < 0 || d.pos + span > d.table_rows))
    return fail(-ERANGE, "rope: positions exceed the table");
  if (d.vc && (!d.kc || !d.v || d.ldv < H * D)) return fail(-EINVAL, "rope_quant: the V cache write needs kc and v rows");
  if (d.kc) {
    if (!d.pos_dev && !d.row_pos && d.pos + span > d.max_seq)
      return fail(-ERANGE, "positions %lld..%lld exceed max_seq=%lld", (long long)d.pos, (long long)(d.pos + span - 1),
                  (long long)d.max_seq);
    if ((d.row_pos || d.seq_rows > 0) && d.slot_stride < H * d.max_seq * D)
      return fail(-EINVAL, "rope_quant: cache slots overlap");
  }
  j = RopeJob{};
  j.x = static_cast<const int16_t*>(d.x);
  j.M = M;
  j.ldx = d.ldx;
  j.table_rows = d.table_rows;
  j.qM = d.qM;
  j.ldv = d.ldv;
  j.max_seq = d.max_seq;
  j.slot_stride = d.slot_stride;
  j.seq_rows = d.seq_rows;
  j.total = M * H * (D / 2);
  j.H = (int)H;
  j.D = (int)D;
  j.pos = (int)d.pos;
  j.qS = (int)d.qS;
  j.cos_tab = static_cast<const int16_t*>(d.cos_tab);
  j.sin_tab = static_cast<const int16_t*>(d.sin_tab);
  j.pos_dev = static_cast<const int32_t*>(d.pos_dev);
  j.row_pos = static_cast<const int32_t*>(d.row_pos);
  j.y = static_cast<int16_t*>(d.y);
  j.yq = static_cast<int8_t*>(d.yq);
  j.kc = static_cast<int8_t*>(d.kc);
  j.v = static_cast<const int8_t*>(d.v);
  j.vc = static_cast<int8_t*>(d.vc);
  return 0;
}

static int rope_launch(const RopeJob& a, const RopeJob& b, void* stream) {
  const int64_t total = a.total + b.total;
  if (total == 0) return 0;
  if (total + 256 < (int64_t)UINT32_MAX)
    hipLaunchKernelGGL(rope_quant_kernel<uint32_t>, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, a, b);
  else
    hipLaunchKernelGGL(rope_quant_kernel<int64_t>, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, a, b);
  LLHIP_LAUNCH_CHECK();
  return 0;
}
}  // namespace llhip

extern "C" {

int llhip_rope_quant(const int16_t* x, int64_t M, int64_t H, int64_t D, int64_t ldx, const int16_t* cos_tab,
                     const int16_t* sin_tab, int64_t table_rows, int64_t pos, const int32_t* pos_dev,
                     const int32_t* row_pos, int16_t* y, int8_t* yq, int64_t qM, int64_t qS, int8_t* kc,
                     const int8_t* v, int64_t ldv, int8_t* vc, int64_t max_seq, int64_t slot_stride, void* stream) {
  const llhip_rope_quant_desc d{x, M, H, D, ldx, cos_tab, sin_tab, table_rows, pos, pos_dev, row_pos, y, yq, qM, qS,
                                kc, v, ldv, vc, max_seq, slot_stride, 0};
  RopeJob a, none{};
  const int rc = rope_job(d, a);
  return rc ? rc : rope_launch(a, none, stream);
}

int llhip_rope_quant2(const llhip_rope_quant_desc* a, const llhip_rope_quant_desc* b, void* stream) {
  if (!a || !b) return fail(-EINVAL, "rope_quant2: null descriptor");
  RopeJob ja, jb;
  int rc = rope_job(*a, ja);
  if (!rc) rc = rope_job(*b, jb);
  return rc ? rc : rope_launch(ja, jb, stream);
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

int llhip_greedy_rows(const int16_t* logits, int64_t rows, int64_t ld, int64_t vocab, int32_t* tokens,
                      int32_t* positions, const int32_t* base, int16_t* ring_rows, int64_t ring_ld,
                      int32_t* ring_tokens, int64_t ring_cap, void* stream) {
  if (rows < 0 || vocab <= 0 || vocab >= (1ll << 30) || ld < (vocab + 1) / 2 * 2 || ring_ld < vocab || ring_cap < 0)
    return fail(-EINVAL, "greedy_rows: bad arguments");
  if (rows == 0) return 0;
  if (!logits || !tokens || !positions || !base || (ring_cap && (!ring_rows || !ring_tokens)))
    return fail(-EINVAL, "greedy_rows: null operand");
  if ((uintptr_t)ring_rows % 16) return fail(-EINVAL, "greedy_rows: misaligned record rows");
  hipLaunchKernelGGL(greedy_rows_kernel, dim3((unsigned)rows), dim3(GR_THREADS), 0, (hipStream_t)stream, logits, ld,
                     vocab, tokens, positions, base, ring_rows, ring_ld, ring_tokens, ring_cap, rows);
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

int llhip_rows_first_mismatch_i16(const int16_t* a, int64_t lda, const int16_t* b, int64_t ldb, int64_t rows,
                                  int64_t cols, int64_t* out, void* stream) {
  if (rows < 0 || cols < 0 || lda < cols || ldb < cols || !out || ((rows && cols) && (!a || !b)))
    return fail(-EINVAL, "rows_first_mismatch: bad arguments");
  hipStream_t s = (hipStream_t)stream;
  unsigned long long* o = reinterpret_cast<unsigned long long*>(out);
  hipLaunchKernelGGL(mismatch_init_kernel, dim3(1), dim3(1), 0, s, o);
  if (rows && cols) {
    const int64_t n = rows * cols;
    hipLaunchKernelGGL(mismatch_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 4096)), dim3(256), 0, s, a, lda,
                       b, ldb, rows, cols, o);
  }
  hipLaunchKernelGGL(mismatch_finish_kernel, dim3(1), dim3(1), 0, s, o);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

int llhip_rows_checksum_i16(const int16_t* x, int64_t ld, int64_t rows, int64_t cols, uint64_t* out, void* stream) {
  if (rows < 0 || cols < 0 || ld < cols || (rows && (!x || !out)) || rows > INT32_MAX)
    return fail(-EINVAL, "rows_checksum: bad arguments");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(row_checksum_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, x, ld, cols, out);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

}  // extern "C"
