// Fused decoder-block kernels of libllhip.  Each kernel computes a run of
// consecutive qgraph ops in one launch and writes every intermediate activation
// those ops name, so its results are those of the separate ops (golden.py:275-314
// executes them one by one):
//
//  attn_in : rmsnorm -> quant -> linear q, k, v (+bias) [-> rmsnorm heads (Qwen3 Q/K norm)]
//            -> rope q, k -> quant q, k -> kv_write
//            One workgroup per head block (H query heads, Hkv key heads, Hkv value heads).
//            The workgroup normalises and quantises the M input rows into LDS, computes the
//            block's D output columns with v_mfma_i32_16x16x64_i8 (K split across waves,
//            partials summed in LDS), then runs the head-local tail: requant, Q/K RMSNorm over
//            the head, RoPE (needs columns i and i + D/2 of the same head), quant and the
//            KV-cache write of the key/value rows.
//  mlp_in  : rmsnorm -> quant -> linear gate (silu) + linear up (mul) -> quant
//            (or the unfused linear g, linear u, silu, mul forms).  One workgroup per 16
//            FFN columns computes the gate and the up tile of those columns.
//  norm_gemv: rmsnorm -> quant -> linear (any epilogue), e.g. the final norm + lm_head.
//
// Decode launches are latency-bound (M = 1, a few MB of weights), so every kernel issues all of
// its independent loads at entry in the order they are needed -- RMSNorm operands, LUTs, the
// weight slice, the epilogue operands -- as branch-free buffer loads (out-of-range lanes read
// zeros), and waits for each group only where it is used: the RMSNorm prologue runs while the
// weights are in flight.  No workgroup depends on another inside a launch (no device-scope
// synchronisation).
#include <algorithm>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {

// ---------------------------------------------------------------------------------------
// RMSNorm + quant prologue (golden.py:124-137, 119-120)
// ---------------------------------------------------------------------------------------

// Rows and 4-element output units of this wave.  With M < nw several waves share a row: each
// computes the row's sum of squares (the row is 2 KiB at most) and applies the scale to its own
// units, so no cross-wave reduction is needed.  With M >= nw wave w takes rows w, w + nw, ...
struct NormMap {
  int m0, step, j, G;  // rows m0, m0 + step, ...; units j*64 + lane + i*G*64
};

__device__ __forceinline__ NormMap norm_map(int M) {
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  NormMap r;
  r.m0 = wave % M;
  if (M < nw) {
    r.step = M;
    r.j = wave / M;
    r.G = (nw - r.m0 + M - 1) / M;
  } else {
    r.step = nw;
    r.j = 0;
    r.G = 1;
  }
  return r;
}

// operands of the wave's first row, loaded at kernel entry
struct NormRegs {
  v4i xs[2];  // 8-element chunks lane and lane + 64 (sum of squares)
  v2i xu, gu; // x and gamma of the first output unit
};

__device__ __forceinline__ void norm_prefetch(const NormQuant& pr, int M, const NormMap& nm, NormRegs& r) {
  const int lane = threadIdx.x & 63, nch = pr.K >> 3, nu = pr.K >> 2;
  const Rsrc xr = rsrc(pr.x, (int64_t)M * pr.ldx * 2), gr = rsrc(pr.gamma, (int64_t)pr.K * 2);
  const uint32_t row = (uint32_t)(nm.m0 * pr.ldx * 2);
  r.xs[0] = ld16(xr, lane < nch ? row + 16 * lane : LD_OOB);
  r.xs[1] = ld16(xr, lane + 64 < nch ? row + 16 * (lane + 64) : LD_OOB);
  const int u = nm.j * 64 + lane;
  r.xu = ld8(xr, u < nu ? row + 8 * u : LD_OOB);
  r.gu = ld8(gr, u < nu ? 8 * u : LD_OOB);
}

__device__ __forceinline__ uint32_t norm_row_inv(const NormQuant& pr, const v4i& xs0, const v4i& xs1) {
  uint64_t ss = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int32_t a = lo16(xs0[j]), c = hi16(xs0[j]);
    ss += (uint32_t)(a * a) + (uint32_t)(c * c);  // each square <= 2^30: the pair fits u32
    a = lo16(xs1[j]);
    c = hi16(xs1[j]);
    ss += (uint32_t)(a * a) + (uint32_t)(c * c);
  }
  return rms_inv(wave_sum_u64(ss), pr.eps_t, pr.C);
}

// normalise + quantise output unit u (elements 4u..4u+3) of row m
__device__ __forceinline__ void norm_apply_unit(const NormQuant& pr, int m, int u, uint32_t inv, const v2i& xu,
                                                const v2i& gu, int8_t* a_lds, int lda, bool write_global) {
  if (u >= (pr.K >> 2)) return;
  const double sy = rms_scale(inv, pr.sh_post), sq = mulshift_scale(pr.Mq, pr.Sq);  // exact forms
  const int16_t y0 = (int16_t)rms_apply_d(lo16(xu.x), lo16(gu.x), sy);
  const int16_t y1 = (int16_t)rms_apply_d(hi16(xu.x), hi16(gu.x), sy);
  const int16_t y2 = (int16_t)rms_apply_d(lo16(xu.y), lo16(gu.y), sy);
  const int16_t y3 = (int16_t)rms_apply_d(hi16(xu.y), hi16(gu.y), sy);
  const uint32_t q = (uint32_t)(uint8_t)mulshift_small_sat(y0, sq, -128.0, 127.0) |
                     ((uint32_t)(uint8_t)mulshift_small_sat(y1, sq, -128.0, 127.0) << 8) |
                     ((uint32_t)(uint8_t)mulshift_small_sat(y2, sq, -128.0, 127.0) << 16) |
                     ((uint32_t)(uint8_t)mulshift_small_sat(y3, sq, -128.0, 127.0) << 24);
  *reinterpret_cast<uint32_t*>(a_lds + m * lda + 4 * u) = q;
  if (write_global) {
    if (pr.h_out) {
      v2i y;
      y.x = pack16(y0, y1);
      y.y = pack16(y2, y3);
      *reinterpret_cast<v2i*>(pr.h_out + (int64_t)m * pr.ldx + 4 * u) = y;
    }
    if (pr.hq_out) *reinterpret_cast<uint32_t*>(pr.hq_out + (int64_t)m * pr.K + 4 * u) = q;
  }
}

// The wave's first row and first unit use the registers loaded at entry in straight-line code,
// so their waits cover those loads only; further rows and units (M > waves, or K > 256 * waves
// sharing a row) load inside loops.
__device__ void norm_quant_rows(const NormQuant& pr, const NormRegs& r, int M, const NormMap& nm, int8_t* a_lds,
                                int lda, bool write_global) {
  const int lane = threadIdx.x & 63, nch = pr.K >> 3, nu = pr.K >> 2;
  const Rsrc xr = rsrc(pr.x, (int64_t)M * pr.ldx * 2), gr = rsrc(pr.gamma, (int64_t)pr.K * 2);
  const int ustep = nm.G * 64;
  {
    const int m = nm.m0;
    const uint32_t row = (uint32_t)(m * pr.ldx * 2);
    const uint32_t inv = norm_row_inv(pr, r.xs[0], r.xs[1]);
    norm_apply_unit(pr, m, nm.j * 64 + lane, inv, r.xu, r.gu, a_lds, lda, write_global);
    for (int u0 = nm.j * 64 + ustep; u0 < nu; u0 += ustep) {
      const int u = u0 + lane;
      const v2i xu = ld8(xr, u < nu ? row + 8 * u : LD_OOB), gu = ld8(gr, u < nu ? 8 * u : LD_OOB);
      norm_apply_unit(pr, m, u, inv, xu, gu, a_lds, lda, write_global);
    }
  }
  for (int m = nm.m0 + nm.step; m < M; m += nm.step) {
    const uint32_t row = (uint32_t)(m * pr.ldx * 2);
    const v4i xs0 = ld16(xr, lane < nch ? row + 16 * lane : LD_OOB);
    const v4i xs1 = ld16(xr, lane + 64 < nch ? row + 16 * (lane + 64) : LD_OOB);
    const uint32_t inv = norm_row_inv(pr, xs0, xs1);
    for (int u0 = nm.j * 64; u0 < nu; u0 += ustep) {
      const int u = u0 + lane;
      const v2i xu = ld8(xr, u < nu ? row + 8 * u : LD_OOB), gu = ld8(gr, u < nu ? 8 * u : LD_OOB);
      norm_apply_unit(pr, m, u, inv, xu, gu, a_lds, lda, write_global);
    }
  }
}

// Rows already quantised by llhip_rmsnorm_quant (multi-row launches): the i8 rows [M][K] are
// loaded at kernel entry (16-byte chunks, PRE_CHUNKS per thread) and staged in LDS.
// Normalising M > 1 rows in every workgroup would repeat the whole row prologue per workgroup.
constexpr int PRE_CHUNKS = 8;

struct PreRows {
  v4i c[PRE_CHUNKS];
};

__device__ __forceinline__ void prerows_load(const NormQuant& pr, int M, PreRows& r) {
  const int nt = blockDim.x, tid = threadIdx.x, total = M * (pr.K >> 4);
  const Rsrc q = rsrc(pr.hq_out, (int64_t)M * pr.K);
#pragma unroll
  for (int i = 0; i < PRE_CHUNKS; ++i) {
    const int c = tid + i * nt;
    r.c[i] = ld16(q, c < total ? 16 * c : LD_OOB);
  }
}

__device__ __forceinline__ void prerows_store(const NormQuant& pr, int M, const PreRows& r, int8_t* a_lds, int lda) {
  const int nt = blockDim.x, tid = threadIdx.x, nch = pr.K >> 4, total = M * nch;
#pragma unroll
  for (int i = 0; i < PRE_CHUNKS; ++i) {
    const int c = tid + i * nt;
    if (c < total) *reinterpret_cast<v4i*>(a_lds + (c / nch) * lda + 16 * (c % nch)) = r.c[i];
  }
  // small workgroups: the chunks beyond the prefetched ones
  const Rsrc q = rsrc(pr.hq_out, (int64_t)M * pr.K);
  for (int c = tid + PRE_CHUNKS * nt; c < total; c += nt)
    *reinterpret_cast<v4i*>(a_lds + (c / nch) * lda + 16 * (c % nch)) = ld16(q, 16 * c);
}

// standalone rmsnorm + quant, one workgroup (256 threads) per row: thread t takes chunk t
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(NormQuant pr) {
  __shared__ uint64_t part[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nch = pr.K >> 3;
  const Rsrc xr = rsrc(pr.x + (int64_t)m * pr.ldx, (int64_t)pr.K * 2), gr = rsrc(pr.gamma, (int64_t)pr.K * 2);
  v4i x[NORM_MAX_K / 8 / 256 + 1], g[NORM_MAX_K / 8 / 256 + 1];
  uint64_t ss = 0;
#pragma unroll
  for (int i = 0; i < NORM_MAX_K / 8 / 256 + 1; ++i) {
    const int c = tid + 256 * i;
    x[i] = ld16(xr, c < nch ? 16 * c : LD_OOB);
    g[i] = ld16(gr, c < nch ? 16 * c : LD_OOB);
  }
#pragma unroll
  for (int i = 0; i < NORM_MAX_K / 8 / 256 + 1; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t a = lo16(x[i][j]), c = hi16(x[i][j]);
      ss += (uint32_t)(a * a) + (uint32_t)(c * c);
    }
  ss = wave_sum_u64(ss);
  if (lane == 0) part[wave] = ss;
  __syncthreads();
  const uint32_t inv = rms_inv(part[0] + part[1] + part[2] + part[3], pr.eps_t, pr.C);
  const double sy = rms_scale(inv, pr.sh_post), sq = mulshift_scale(pr.Mq, pr.Sq);  // exact forms
#pragma unroll
  for (int i = 0; i < NORM_MAX_K / 8 / 256 + 1; ++i) {
    const int c = tid + 256 * i;
    if (c >= nch) break;
    v4i y;
    uint32_t qw[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int16_t y0 = (int16_t)rms_apply_d(lo16(x[i][j]), lo16(g[i][j]), sy);
      const int16_t y1 = (int16_t)rms_apply_d(hi16(x[i][j]), hi16(g[i][j]), sy);
      y[j] = pack16(y0, y1);
      const uint32_t q0 = (uint8_t)mulshift_small_sat(y0, sq, -128.0, 127.0);
      const uint32_t q1 = (uint8_t)mulshift_small_sat(y1, sq, -128.0, 127.0);
      qw[j >> 1] |= (q0 | (q1 << 8)) << (16 * (j & 1));
    }
    if (pr.h_out) *reinterpret_cast<v4i*>(pr.h_out + (int64_t)m * pr.ldx + 8 * c) = y;
    if (pr.hq_out) {
      v2i q2;
      q2.x = (int)qw[0];
      q2.y = (int)qw[1];
      *reinterpret_cast<v2i*>(pr.hq_out + (int64_t)m * pr.K + 8 * c) = q2;
    }
  }
}

// SIG table (258 u16 = 129 dwords) staged into LDS by one wave (threads first..first+63, wave 0
// by default): three dword loads per lane at kernel entry, stored once the prologue waits anyway
struct SigRegs {
  uint32_t w[3];
};

__device__ __forceinline__ void sig_prefetch(SigRegs& r, int first = 0) {
  const int t = (int)threadIdx.x - first;
  const Rsrc sr = rsrc(kSig, sizeof(kSig));
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int idx = t + 64 * i;
    r.w[i] = (uint32_t)ld4(sr, (t >= 0 && t < 64 && idx < 129) ? 4 * idx : LD_OOB);
  }
}

// sig_store into a 192-dword array: every lane stores its three dwords (zeros past the table), so
// no load is used under a condition (the compiler would move it there, behind a wait)
__device__ __forceinline__ void sig_store192(const SigRegs& r, uint32_t* sig32, int first) {
  const int t = (int)threadIdx.x - first;
  if (t >= 0 && t < 64) {
#pragma unroll
    for (int i = 0; i < 3; ++i) sig32[t + 64 * i] = r.w[i];
  }
}

__device__ __forceinline__ void sig_store(const SigRegs& r, uint32_t* sig32, int first = 0) {
  const int t = (int)threadIdx.x - first;
  if (t >= 0 && t < 64) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
      if (t + 64 * i < 129) sig32[t + 64 * i] = r.w[i];
  }
}

// ---------------------------------------------------------------------------------------
// decode-chain prologue (one row): the row x finishes the previous projection, then RMSNorm and
// quant of x (golden.py:316-342 resadd epilogue, then 124-137 and 119-120)
// ---------------------------------------------------------------------------------------
// The previous launch left that projection (linear W, epilogue resadd with residual aux) as exact
// int32 partial sums in R accumulator rows; x[n] = sat16(sat16(mulshift(sum_r acc[r][n] + bias[n],
// M_n, S_n)) + aux[n]).  Without partial sums x is read from memory (the first layer).  Thread t
// owns the 4-element unit t of the row; every operand is loaded at kernel entry (null operands
// read zeros), and the sum of squares is one block reduction.
struct ResidArgs {
  const int32_t* acc;  // [R][K] int32 partial sums, or null (x is read from pre.x)
  const int32_t* rq;   // [K][2] requant pairs of the projection
  const int32_t* bias; // [K] or null
  const int16_t* aux;  // [K] residual
  int16_t* x_out;      // [K] the finished row, written by workgroup 0
  int R;
};
constexpr int RESID_MAXR = 8;

struct ResidRegs {
  v4i acc[RESID_MAXR];
  v4i rq[2];
  v4i bias;
  v2i x, g;
};

__device__ __forceinline__ void resid_prefetch(const NormQuant& pr, const ResidArgs& ra, ResidRegs& r) {
  const int u = threadIdx.x, K = pr.K;
  const bool in = u < (K >> 2);
  const bool fin = ra.acc != nullptr;
#pragma unroll
  for (int i = 0; i < RESID_MAXR; ++i) r.acc[i] = v4i{0, 0, 0, 0};
  r.rq[0] = r.rq[1] = r.bias = v4i{0, 0, 0, 0};
  r.x = r.g = v2i{0, 0};
  // waves past the row's units issue nothing (a load instruction costs address-unit cycles for
  // all 64 lanes, in range or not)
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 256 >= K) return;
  const Rsrc ar = rsrc(ra.acc, (int64_t)ra.R * K * 4);
#pragma unroll
  for (int i = 0; i < RESID_MAXR; ++i)
    if (i < ra.R) r.acc[i] = ld16(ar, in ? (uint32_t)((i * K + 4 * u) * 4) : LD_OOB);
  const Rsrc qr = rsrc(fin ? ra.rq : nullptr, (int64_t)K * 8);
  r.rq[0] = ld16(qr, in ? 32u * u : LD_OOB);
  r.rq[1] = ld16(qr, in ? 32u * u + 16u : LD_OOB);
  r.bias = ld16(rsrc(fin ? ra.bias : nullptr, (int64_t)K * 4), in ? 16u * u : LD_OOB);
  // x: the residual when finishing, else the row itself
  r.x = ld8(rsrc(fin ? (const void*)ra.aux : (const void*)pr.x, (int64_t)K * 2), in ? 8u * u : LD_OOB);
  r.g = ld8(rsrc(pr.gamma, (int64_t)K * 2), in ? 8u * u : LD_OOB);
}

// thread u's four values of the row x (finished from the partial sums, or as read) and their sum of
// squares
__device__ __forceinline__ uint64_t resid_row(const ResidArgs& ra, const ResidRegs& r, int32_t xv[4]) {
  xv[0] = lo16(r.x.x);
  xv[1] = hi16(r.x.x);
  xv[2] = lo16(r.x.y);
  xv[3] = hi16(r.x.y);
  if (ra.acc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int32_t s = 0;
#pragma unroll
      for (int i = 0; i < RESID_MAXR; ++i) s += r.acc[i][j];  // |sum| < 2^31: an exact K-split of one dot product
      const int32_t M = r.rq[j >> 1][2 * (j & 1)], S = r.rq[j >> 1][2 * (j & 1) + 1];
      const int64_t t = sat16(mulshift((int64_t)s + r.bias[j], (int64_t)M, S));
      xv[j] = (int32_t)sat16(t + xv[j]);
    }
  }
  uint64_t ss = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) ss += (uint64_t)(uint32_t)(xv[j] * xv[j]);
  return ss;
}

// RMSNorm (reciprocal inv) and quant of thread u's four values into a_lds (i8); workgroup 0 writes
// x (when finishing), h_out and hq_out
__device__ __forceinline__ void resid_apply(const NormQuant& pr, const ResidArgs& ra, const ResidRegs& r,
                                            const int32_t xv[4], uint32_t inv, int8_t* a_lds, bool write_global) {
  const int u = threadIdx.x;
  if (u >= (pr.K >> 2)) return;
  const int32_t g[4] = {lo16(r.g.x), hi16(r.g.x), lo16(r.g.y), hi16(r.g.y)};
  // double-precision forms of rms_apply and of the quant's mulshift (exact for these ranges)
  const double sy = rms_scale(inv, pr.sh_post), sq = mulshift_scale(pr.Mq, pr.Sq);
  int16_t y[4];
  uint32_t q = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    y[j] = (int16_t)rms_apply_d(xv[j], g[j], sy);
    q |= (uint32_t)(uint8_t)mulshift_small_sat(y[j], sq, -128.0, 127.0) << (8 * j);
  }
  *reinterpret_cast<uint32_t*>(a_lds + 4 * u) = q;
  if (write_global) {
    if (ra.acc && ra.x_out) {
      v2i xo;
      xo.x = pack16(xv[0], xv[1]);
      xo.y = pack16(xv[2], xv[3]);
      *reinterpret_cast<v2i*>(ra.x_out + 4 * u) = xo;
    }
    if (pr.h_out) {
      v2i yo;
      yo.x = pack16(y[0], y[1]);
      yo.y = pack16(y[2], y[3]);
      *reinterpret_cast<v2i*>(pr.h_out + 4 * u) = yo;
    }
    if (pr.hq_out) *reinterpret_cast<uint32_t*>(pr.hq_out + 4 * u) = q;
  }
}

// x, RMSNorm, quant of the row into a_lds (i8); workgroup 0 writes x (when finishing), h_out and
// hq_out.  red64 is LDS for one u64 per wave.  Ends with a barrier.
__device__ __forceinline__ void resid_norm_quant(const NormQuant& pr, const ResidArgs& ra, const ResidRegs& r,
                                                 int8_t* a_lds, bool write_global, uint64_t* red64) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int32_t xv[4];
  uint64_t ss = wave_sum_u64(resid_row(ra, r, xv));
  if (lane == 0) red64[wave] = ss;
  __syncthreads();
  uint64_t tot = 0;
  for (int w = 0; w < nw; ++w) tot += red64[w];
  resid_apply(pr, ra, r, xv, rms_inv(tot, pr.eps_t, pr.C), a_lds, write_global);
  __syncthreads();
}

// zero n int32 accumulators (the next projection's) from one workgroup
__device__ __forceinline__ void zero_rows(int32_t* p, int n) {
  if (!p) return;
  for (int i = 4 * threadIdx.x; i < n; i += 4 * blockDim.x) {
    if (i + 4 <= n) *reinterpret_cast<v4i*>(p + i) = v4i{0, 0, 0, 0};
    else
      for (int j = i; j < n; ++j) p[j] = 0;
  }
}

// ---------------------------------------------------------------------------------------
// weight slices: W [N][K] i8, 16 columns x one wave's K steps
// ---------------------------------------------------------------------------------------
// The first PF 64-deep K steps of a wave's slice are loaded at kernel entry; longer slices stream
// the rest four steps at a time.  Lane (col, kg) holds K bytes [s*64 + kg*16, +16) of column col.
constexpr int PF = 8;

// NP: the K steps loaded at entry (the launch sizes it to the steps of a wave's K range, so no load
// instruction is spent on steps past the range)
template <int NP = PF>
struct WSlice {
  v4i w[NP];
  uint32_t rowoff;
  int s0, s1, kg;
};

template <int NP>
__device__ __forceinline__ void wslice_prefetch(WSlice<NP>& ws, Rsrc wr, int n, int K, int kg, int s0, int s1) {
  ws.rowoff = (uint32_t)n * (uint32_t)K;  // rows n >= N fall past the range and read zeros
  ws.s0 = s0;
  ws.s1 = s1;
  ws.kg = kg;
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int k = (s0 + u) * 64 + kg * 16;
    ws.w[u] = ld16(wr, (s0 + u < s1 && k < K) ? ws.rowoff + k : LD_OOB);
  }
}

// 16x16 partial tile of the slice; A rows from LDS.  A rows >= M are read from row M - 1: output
// row m depends only on A row m, so those rows only produce discarded outputs.  Steps past the
// slice have zero weights, so their A reads only need to stay inside the LDS rows.
template <int NP>
__device__ __forceinline__ v4i wslice_mfma(const WSlice<NP>& ws, Rsrc wr, const int8_t* a_lds, int lda, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int8_t* arow = a_lds + min(lane & 15, M - 1) * lda;
  v4i acc = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int k = min((ws.s0 + u) * 64 + ws.kg * 16, K - 16);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const v4i*>(arow + k), ws.w[u], acc, 0, 0, 0);
  }
  for (int s = ws.s0 + NP; s < ws.s1; s += 4) {
    v4i b[4], a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = (s + u) * 64 + ws.kg * 16;
      b[u] = ld16(wr, (s + u < ws.s1 && k < K) ? ws.rowoff + k : LD_OOB);
      a[u] = *reinterpret_cast<const v4i*>(arow + min(k, K - 16));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
  }
  return acc;
}

__device__ __forceinline__ void split_range(int steps, int parts, int idx, int& s0, int& s1) {
  const int spw = (steps + parts - 1) / parts;
  s0 = min(idx * spw, steps);
  s1 = min(s0 + spw, steps);
}

__device__ __forceinline__ void v4_add(v4i& a, const v4i& b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

// ---------------------------------------------------------------------------------------
// attn_in
// ---------------------------------------------------------------------------------------
struct AttnInArgs {
  NormQuant pre;
  const int8_t* W[3];
  const int32_t* rq[3];
  const int32_t* bias[3];
  void* lin_out[3];  // q i16 [M][H*D], k i16 [M][Hkv*D], v i8 [M][Hkv*D]
  const int16_t* nrm_gamma[2];
  int16_t* nrm_out[2];
  int64_t nrm_eps[2], nrm_C[2], nrm_sh[2];
  const int16_t* cos_tab;
  const int16_t* sin_tab;
  const int32_t* pos_dev;
  const int32_t* row_pos;  // per-row positions (row m in cache slot m), or null
  int64_t slot_stride;
  int16_t* rope_out[2];
  int8_t* quant_out[2];
  int64_t quant_M[2], quant_S[2];
  int8_t* kc;
  int8_t* vc;
  int64_t max_seq;
  int M, H, Hkv, D, K, pos, KS, has_norm;
  // decode chain (RESID kernels, M = 1): the row from the previous projection's partial sums, and
  // the accumulators this launch clears for the attention's output projection
  ResidArgs res;
  int32_t* zero;
  int zero_n;
};

// per-role kernel arguments chosen by scalar selects of the three values (an indexed read of the
// argument array would wait on the role before the load could issue)
template <class T>
__device__ __forceinline__ T pick3(int role, const T (&v)[3]) {
  const T a = v[0], b = v[1], c = v[2];
  return role == 0 ? a : (role == 1 ? b : c);
}

// SPL > 1 (decode chain, no head norm): SPL workgroups per head block, workgroup s taking the
// 16-column tiles t with t % SPL == s -- a tile and its RoPE partner t + D/32 fall in the same
// workgroup when (D / 32) % SPL == 0 -- so each streams 1/SPL of the head's weights.
template <int MAXW, bool RESID, int SPL = 1, int PFN = PF>
__global__ __launch_bounds__(64 * MAXW) void attn_in_kernel(AttnInArgs p) {
  kernarg_warm<sizeof(AttnInArgs)>();
  extern __shared__ __attribute__((aligned(16))) int8_t dyn[];
  __shared__ v4i red[MAXW][64];
  __shared__ int32_t rowpos[16];
  __shared__ uint64_t red64[MAXW];
  const int lda = p.K + 16;
  int8_t* a_lds = dyn;                                                         // [M][lda] i8
  int32_t* hres = reinterpret_cast<int32_t*>(dyn + ((p.M * lda + 15) & ~15));  // [M][D] i32

  const int b = blockIdx.x;
  const int bh = b / SPL, sp = b % SPL;  // head block, its tile share
  const int role = bh < p.H ? 0 : (bh < p.H + p.Hkv ? 1 : 2);
  const int hh = role == 0 ? bh : (role == 1 ? bh - p.H : bh - p.H - p.Hkv);
  const int D = p.D, M = p.M;
  const int Nrole = (role == 0 ? p.H : p.Hkv) * D;
  const int base = hh * D;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int tiles = (D >> 4) / SPL;  // 16-column tiles of this workgroup
  const int DW = D / SPL;            // its columns
  // head column of this workgroup's column lc: tile (lc / 16) * SPL + sp
  auto gcol = [&](int lc) { return 16 * ((lc >> 4) * SPL + sp) + (lc & 15); };

  // kernel entry, in order of use: the device position, RMSNorm operands, weight slice, epilogue
  // operands of this thread's column, head-norm gamma.  The position is a vector load issued
  // first (the previous launch wrote it, so it comes from memory): it has arrived once the
  // RMSNorm operands have, and only then are the RoPE factors at that position requested.
  const int32_t posv = ld4(rsrc(p.pos_dev, 4), 0);
  // per-row positions: the row of this thread's RoPE pair and row tid (staged in LDS for the tail)
  const int half = D >> 1;
  const int jrope = gcol(tid % (half / SPL)), mrope = tid / (half / SPL);
  int32_t rp_rope = 0, rp_own = 0;
  if (p.row_pos) {  // (a load instruction costs address-unit cycles even when it reads nothing)
    const Rsrc rpr = rsrc(p.row_pos, 4 * M);
    rp_rope = ld4(rpr, mrope < M ? 4 * mrope : LD_OOB);
    rp_own = ld4(rpr, tid < M ? 4 * tid : LD_OOB);
  }
  issue_fence();
  const NormMap nm = norm_map(M);
  NormRegs nr;
  PreRows pq;
  ResidRegs rr;
  if constexpr (RESID)
    resid_prefetch(p.pre, p.res, rr);
  else if (p.pre.prequant)
    prerows_load(p.pre, M, pq);
  else
    norm_prefetch(p.pre, M, nm, nr);
  issue_fence();
  const Rsrc wr = rsrc(pick3(role, p.W), (int64_t)Nrole * p.K);
  WSlice<PFN> ws;
  {
    const int t = wave % tiles, ks = wave / tiles;
    int s0, s1;
    split_range((p.K + 63) >> 6, p.KS, ks, s0, s1);
    wslice_prefetch(ws, wr, base + (t * SPL + sp) * 16 + (lane & 15), p.K, lane >> 4, s0, s1);
  }
  issue_fence();
  const int dcol = gcol(tid % DW);  // blockDim is a multiple of DW: each thread owns one column in the tail
  const int ncol = base + dcol;
  const v2i rq = ld8(rsrc(pick3(role, p.rq), (int64_t)Nrole * 8), 8 * ncol);
  const int32_t bias = ld4(rsrc(pick3(role, p.bias), (int64_t)Nrole * 4), 4 * ncol);
  const bool hn = SPL == 1 && p.has_norm && role < 2;  // split heads are never normed (host)
  int32_t hg[4] = {0, 0, 0, 0};  // head-norm gamma of dims lane + 64 i (the per-row norm runs wave-wide)
  if (hn) {
    const Rsrc gr = rsrc(role == 0 ? p.nrm_gamma[0] : p.nrm_gamma[1], (int64_t)D * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) hg[i] = ld2s(gr, lane + 64 * i < D ? 2 * (lane + 64 * i) : LD_OOB);
  }
  issue_fence();

  if constexpr (RESID) {
    if (b == 0) zero_rows(p.zero, p.zero_n);
    resid_norm_quant(p.pre, p.res, rr, a_lds, b == 0, red64);
  } else if (p.pre.prequant) {
    prerows_store(p.pre, M, pq, a_lds, lda);
  } else {
    norm_quant_rows(p.pre, nr, M, nm, a_lds, lda, b == 0);
  }
  const int pos0 = p.pos_dev ? __builtin_amdgcn_readfirstlane(posv) : p.pos;
  const bool rows = p.row_pos != nullptr;
  if (tid < M) rowpos[tid] = rows ? rp_own : pos0 + tid;
  int32_t c0 = 0, s0r = 0;
  {
    const int pr = rows ? rp_rope : pos0 + mrope;
    const bool rok = role < 2 && mrope < M && pr >= 0 && pr < p.max_seq;
    const int64_t tab = (int64_t)p.max_seq * half * 2;
    const uint32_t off = rok ? (uint32_t)(((int64_t)pr * half + jrope) * 2) : LD_OOB;
    c0 = ld2s(rsrc(p.cos_tab, tab), off);
    s0r = ld2s(rsrc(p.sin_tab, tab), off);
  }
  issue_fence();
  __syncthreads();
  red[wave][lane] = wslice_mfma(ws, wr, a_lds, lda, M, p.K);
  __syncthreads();
  if (wave < tiles) {
    v4i acc = red[wave][lane];
    for (int ks = 1; ks < p.KS; ++ks) v4_add(acc, red[wave + ks * tiles][lane]);
    const int col = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * kg + r;
      if (m < M) hres[m * D + (wave * SPL + sp) * 16 + col] = acc[r];
    }
  }
  __syncthreads();

  const int rstep = blockDim.x / DW;
  if (role == 2) {  // v: requant8 -> v activation and V cache
    for (int m = tid / DW; m < M; m += rstep) {
      const int8_t y = (int8_t)sat8(mulshift((int64_t)hres[m * D + dcol] + bias, rq.x, rq.y));
      static_cast<int8_t*>(p.lin_out[2])[(int64_t)m * Nrole + ncol] = y;
      const int pm = rowpos[m];
      if (pm >= 0 && pm < p.max_seq)  // device positions are checked by the caller; never write past a cache
        p.vc[(rows ? m * p.slot_stride : 0) + ((int64_t)hh * p.max_seq + pm) * D + dcol] = y;
    }
    return;
  }
  // q / k: requant16 -> activation; head values kept in hres as int32
  for (int m = tid / DW; m < M; m += rstep) {
    const int16_t y = (int16_t)sat16(mulshift((int64_t)hres[m * D + dcol] + bias, rq.x, rq.y));
    static_cast<int16_t*>(p.lin_out[role])[(int64_t)m * Nrole + ncol] = y;
    hres[m * D + dcol] = y;
  }
  __syncthreads();
  if (hn) {  // RMSNorm over each D-wide head (golden.py:287-293, heads > 1)
    const int nw = blockDim.x >> 6;
    for (int m = wave; m < M; m += nw) {
      uint64_t ss = 0;
      for (int d = lane; d < D; d += 64) ss += (uint64_t)(uint32_t)(hres[m * D + d] * hres[m * D + d]);
      ss = wave_sum_u64(ss);
      const uint32_t inv = rms_inv(ss, (uint32_t)p.nrm_eps[role], (uint32_t)p.nrm_C[role]);
      const double sy = rms_scale(inv, (int)p.nrm_sh[role]);  // exact double form of rms_apply
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d >= D) break;
        const int16_t y = (int16_t)rms_apply_d(hres[m * D + d], hg[i], sy);
        p.nrm_out[role][(int64_t)m * Nrole + base + d] = y;
        hres[m * D + d] = y;
      }
    }
    __syncthreads();
  }
  // RoPE (golden.py:141-158) -> quant (golden.py:119-120) -> K cache for keys: the rotation's sums
  // in 64-bit (x and the table entries are i16, so a sum reaches 2^31 when all four are -32768), and
  // the quant's mulshift of an i16 is exact in double (mulshift_small_sat)
  const double sq = mulshift_scale(p.quant_M[role], (int)p.quant_S[role]);
  for (int m = mrope; m < M; m += blockDim.x / (half / SPL)) {
    int32_t c = c0, s = s0r;
    const int pm = rowpos[m];
    if (pm < 0 || pm >= p.max_seq) continue;
    if (m != mrope) {
      c = p.cos_tab[(int64_t)pm * half + jrope];
      s = p.sin_tab[(int64_t)pm * half + jrope];
    }
    const int j = jrope;
    const int32_t x1 = hres[m * D + j], x2 = hres[m * D + half + j];
    const int16_t y1 = (int16_t)sat16(rshr((int64_t)x1 * c - (int64_t)x2 * s, 14));
    const int16_t y2 = (int16_t)sat16(rshr((int64_t)x2 * c + (int64_t)x1 * s, 14));
    const int64_t o = (int64_t)m * Nrole + base;
    p.rope_out[role][o + j] = y1;
    p.rope_out[role][o + half + j] = y2;
    const int8_t q1 = (int8_t)mulshift_small_sat(y1, sq, -128.0, 127.0);
    const int8_t q2 = (int8_t)mulshift_small_sat(y2, sq, -128.0, 127.0);
    p.quant_out[role][o + j] = q1;
    p.quant_out[role][o + half + j] = q2;
    if (role == 1) {
      int8_t* kr = p.kc + (rows ? m * p.slot_stride : 0) + ((int64_t)hh * p.max_seq + pm) * D;
      kr[j] = q1;
      kr[half + j] = q2;
    }
  }
}

// ---------------------------------------------------------------------------------------
// mlp_in
// ---------------------------------------------------------------------------------------
struct MlpInArgs {
  NormQuant pre;
  const int8_t* Wg;
  const int8_t* Wu;
  const int32_t* rqg;
  const int32_t* rqu;
  const int32_t* bg;
  const int32_t* bu;
  int16_t* g_out;  // unfused graphs only
  int16_t* u_out;  // unfused graphs only
  int16_t* sg_out;
  int16_t* f_out;
  int8_t* fq_out;
  int64_t silu_Mi, fq_M;
  int silu_Si, silu_sh, mul_sh, fq_S;
  int M, N, K, KS;
  // decode chain (dec_mlp_kernel, M = 1): the row from the output projection's partial sums, and
  // the down projection's partial sums of the workgroup's FFN columns j: wd_acc[r][n] +=
  // sum_j fq[j] * Wd[n][j], read from the panel wdp[b][n][i] = Wd[n][16 b + i]
  ResidArgs res;
  const int8_t* wdp;
  int32_t* wd_acc;
  int wd_R, wd_N;
  // dec_mlp_kernel's column assignment: workgroup b < W owns FFN tile b (columns 16b..16b+15) and
  // at most one tail group of tail_gw columns of the tiles W.. (see dec_tail_group)
  int tail_tiles, tail_gw;
};

constexpr int WD_PF = 4;  // down-projection panel columns per thread loaded at kernel entry

template <int MAXW>
__global__ __launch_bounds__(64 * MAXW) void mlp_in_kernel(MlpInArgs p) {
  kernarg_warm<sizeof(MlpInArgs)>();
  extern __shared__ __attribute__((aligned(16))) int8_t dyn[];
  __shared__ v4i red[MAXW][64];
  __shared__ uint32_t sig32[129];
  const int lda = p.K + 16;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int col = lane & 15, kg = lane >> 4;
  const int n = blockIdx.x * 16 + col;

  const NormMap nm = norm_map(p.M);
  NormRegs nr;
  PreRows pq;
  if (p.pre.prequant)
    prerows_load(p.pre, p.M, pq);
  else
    norm_prefetch(p.pre, p.M, nm, nr);
  issue_fence();
  SigRegs sr;
  sig_prefetch(sr);
  issue_fence();
  const int up = wave >= p.KS;  // waves [0, KS): gate, [KS, 2KS): up
  const Rsrc wr = rsrc(up ? p.Wu : p.Wg, (int64_t)p.N * p.K);
  WSlice<> ws;
  {
    int s0, s1;
    split_range((p.K + 63) >> 6, p.KS, up ? wave - p.KS : wave, s0, s1);
    wslice_prefetch(ws, wr, n, p.K, kg, s0, s1);
  }
  issue_fence();
  const uint32_t o8 = n < p.N ? 8 * n : LD_OOB, o4 = n < p.N ? 4 * n : LD_OOB;
  v2i rg = ld8(rsrc(p.rqg, (int64_t)p.N * 8), o8);
  v2i ru = ld8(rsrc(p.rqu, (int64_t)p.N * 8), o8);
  int32_t bgv = ld4(rsrc(p.bg, (int64_t)p.N * 4), o4);
  int32_t buv = ld4(rsrc(p.bu, (int64_t)p.N * 4), o4);
  issue_fence();

  if (p.pre.prequant)
    prerows_store(p.pre, p.M, pq, dyn, lda);
  else
    norm_quant_rows(p.pre, nr, p.M, nm, dyn, lda, blockIdx.x == 0);
  sig_store(sr, sig32);
  __syncthreads();
  red[wave][lane] = wslice_mfma(ws, wr, dyn, lda, p.M, p.K);
  __syncthreads();
  if (wave == 0) {
    // the requant operands are used from here on (the compiler may not widen them earlier, which
    // would wait for every load before the prologue)
    asm volatile("" : "+v"(rg), "+v"(ru), "+v"(bgv), "+v"(buv));
    v4i ag = red[0][lane], au = red[p.KS][lane];
    for (int ks = 1; ks < p.KS; ++ks) {
      v4_add(ag, red[ks][lane]);
      v4_add(au, red[p.KS + ks][lane]);
    }
    const uint16_t* sig = reinterpret_cast<const uint16_t*>(sig32);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * kg + r;
      if (m >= p.M || n >= p.N) continue;
      const int64_t o = (int64_t)m * p.N + n;
      const int64_t tg = sat16(mulshift((int64_t)ag[r] + bgv, rg.x, rg.y));
      const int64_t tu = sat16(mulshift((int64_t)au[r] + buv, ru.x, ru.y));
      if (p.g_out) p.g_out[o] = (int16_t)tg;
      if (p.u_out) p.u_out[o] = (int16_t)tu;
      const int64_t sg = silu16_lds(tg, p.silu_Mi, p.silu_Si, p.silu_sh, sig);
      const int64_t f = sat16(rshr(tu * sg, p.mul_sh));
      p.sg_out[o] = (int16_t)sg;
      p.f_out[o] = (int16_t)f;
      p.fq_out[o] = (int8_t)sat8(mulshift(f, p.fq_M, p.fq_S));
    }
  }
}

// ---------------------------------------------------------------------------------------
// dec_mlp (decode chain, one row): mlp_in over the FFN columns, then the down projection's partial
// sums of those columns.  The work of a workgroup is split over two sets of waves.  Waves 0-3 (the
// norm waves) finish the output projection's row from its partial sums, normalise and quantise it
// into LDS; waves 4-7 (the weight waves) stream the gate (waves 4, 5: the two K halves) and up
// (6, 7) weights and the down-projection panel.  A wave that issues a long run of loads cannot
// pass a workgroup barrier before the last one is issued, so the norm waves meet through an LDS
// counter instead.  Then the weight waves' MFMAs, wave 0's requant / SiLU / mul / quant epilogue,
// and the weight waves' down-projection partial sums (the accumulator layout of the mlp_in decode
// form: workgroup b adds into row b % R).
// Columns: with more 16-column tiles than CUs, one tile per workgroup would put two workgroups on
// some CUs and the launch would last twice as long there.  So the grid is W = #CUs workgroups,
// workgroup b owns tile b, and the tiles past W are cut into groups of gw = 4, 8 or 16 columns
// (bytes 4i.. of a panel row) handed to one workgroup each.  The groups of one tile go to
// workgroups of one XCD (workgroup b runs on XCD b % 8), which then read each panel line once
// through their shared L2.
// ---------------------------------------------------------------------------------------
constexpr int DM_THREADS = 512;  // 4 norm waves + 4 weight waves

// waves [0, n) meet without the others: each adds one to *cnt (zeroed before the workgroup's first
// barrier, and only these waves add to it) and waits until all n have.  Only LDS is ordered (the
// LDS performs one wave's operations in issue order): a release/acquire pair would also wait for
// every global load in flight, which is what the meeting must not do.
__device__ __forceinline__ void wave_group_meet(int* cnt, int n) {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS writes before the add
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < n) __builtin_amdgcn_s_sleep(1);
  __asm__ volatile("" ::: "memory");  // LDS reads of the others' values stay after the wait
}

// the tail group of workgroup b: its first column (or -1: none).  Tile u of the tail (u < tiles)
// has 16 / gw groups i, held by workgroup (u % 8) + 8 * ((u / 8) * (16 / gw) + i).
__host__ __device__ __forceinline__ int dec_tail_group(int b, int W, int tiles, int gw) {
  if (tiles <= 0) return -1;
  const int per = 16 / gw, x = b % 8, slot = b / 8;
  const int u = (slot / per) * 8 + x, i = slot % per;
  return u < tiles ? 16 * (W + u) + gw * i : -1;
}

template <int GW>
__global__ __launch_bounds__(DM_THREADS) void dec_mlp_kernel(MlpInArgs p) {
  kernarg_warm<sizeof(MlpInArgs)>();
  extern __shared__ __attribute__((aligned(16))) int8_t dyn[];  // the quantised row
  __shared__ v4i red[2][4][64];  // [main, tail][weight wave] MFMA tiles
  __shared__ uint32_t sig32[192];
  __shared__ uint64_t red64[4];
  __shared__ int meet;
  __shared__ __attribute__((aligned(16))) int8_t fq16[2][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int col = lane & 15, kg = lane >> 4;
  const int W = (int)gridDim.x, gw = GW;
  const int t0 = dec_tail_group((int)blockIdx.x, W, p.tail_tiles, GW);  // first tail column, or -1
  if (tid == 0) meet = 0;
  __syncthreads();  // no load has been issued yet: every wave is here at once

  WSlice<> ws[2];
  Rsrc wr;
  v4i wdv[WD_PF];     // weight waves: their first panel rows of the main tile
  v4i wdt[WD_PF];     // ... and the tail group's bytes of the tail tile's rows
  v2i rq{0, 0};       // wave 0: the epilogue's requant pair and bias for gate (g) and up (u)
  v2i rqu{0, 0};
  int32_t bgv = 0, buv = 0;
  // wave 0's epilogue lanes: kg 0 = the main tile's column col, kg 1 = the tail group's column col
  const int en = kg == 0 ? (int)blockIdx.x * 16 + col : (kg == 1 && t0 >= 0 && col < gw ? t0 + col : p.N);
  // Load order matters: a wave's loads complete in issue order, so whatever a wave issues before
  // (or, through a branch the wait counts cannot see past, beside) the loads it needs first is
  // waited for too.  The norm waves issue their row operands, then wave 0's epilogue operands
  // (the other norm waves issue the same loads out of range, so every norm wave has the same
  // count in flight); the SIG table is the last load of wave 4.
  if (wave < 4) {
    ResidRegs rr;
    resid_prefetch(p.pre, p.res, rr);
    issue_fence();
    {
      const bool mine = wave == 0 && en < p.N;
      const uint32_t o8 = mine ? 8 * en : LD_OOB, o4 = mine ? 4 * en : LD_OOB;
      rq = ld8(rsrc(p.rqg, (int64_t)p.N * 8), o8);
      rqu = ld8(rsrc(p.rqu, (int64_t)p.N * 8), o8);
      bgv = ld4(rsrc(p.bg, (int64_t)p.N * 4), o4);
      buv = ld4(rsrc(p.bu, (int64_t)p.N * 4), o4);
    }
    issue_fence();
    int32_t xv[4];
    const uint64_t ss = wave_sum_u64(resid_row(p.res, rr, xv));
    if (lane == 0) red64[wave] = ss;
    wave_group_meet(&meet, 4);
    const uint32_t inv = rms_inv(red64[0] + red64[1] + red64[2] + red64[3], p.pre.eps_t, p.pre.C);
    resid_apply(p.pre, p.res, rr, xv, inv, dyn, blockIdx.x == 0);
  } else {
    const int wi = wave - 4;
    wr = rsrc(wi >= 2 ? p.Wu : p.Wg, (int64_t)p.N * p.K);
    int s0, s1;
    split_range((p.K + 63) >> 6, 2, wi & 1, s0, s1);
    wslice_prefetch(ws[0], wr, (int)blockIdx.x * 16 + col, p.K, kg, s0, s1);
    // tail lanes past the group read zeros (row N is past the weights)
    wslice_prefetch(ws[1], wr, t0 >= 0 && col < gw ? t0 + col : p.N, p.K, kg, t0 >= 0 ? s0 : s1, s1);
    issue_fence();
    const int64_t rows = (int64_t)((p.N + 15) / 16) * p.wd_N * 16;
    const Rsrc dr = rsrc(p.wdp, rows);
    const int64_t tbase = t0 >= 0 ? (int64_t)(t0 >> 4) * p.wd_N * 16 + (t0 & 15) : 0;
#pragma unroll
    for (int i = 0; i < WD_PF; ++i) {
      const int c = tid - 256 + 256 * i;
      const bool in = c < p.wd_N;
      wdv[i] = ld16(dr, in ? (uint32_t)(((int64_t)blockIdx.x * p.wd_N + c) * 16) : LD_OOB);
      const uint32_t to = (in && t0 >= 0) ? (uint32_t)(tbase + 16 * (int64_t)c) : LD_OOB;
      if constexpr (GW == 16) {
        wdt[i] = ld16(dr, to);
      } else if constexpr (GW == 8) {
        const v2i w2 = ld8(dr, to);
        wdt[i] = v4i{w2.x, w2.y, 0, 0};
      } else {
        wdt[i] = v4i{ld4(dr, to), 0, 0, 0};
      }
    }
    issue_fence();
    SigRegs sr;
    sig_prefetch(sr, 256);
    issue_fence();
    sig_store192(sr, sig32, 256);
  }
  __syncthreads();
  if (wave >= 4) {
    red[0][wave - 4][lane] = wslice_mfma(ws[0], wr, dyn, p.K + 16, 1, p.K);
    if (t0 >= 0) red[1][wave - 4][lane] = wslice_mfma(ws[1], wr, dyn, p.K + 16, 1, p.K);
  }
  __syncthreads();
  if (wave == 0 && kg < 2) {
    // the requant operands are used from here on: the compiler may not widen them (and wait for
    // their loads, which queue behind the weights) while the norm waves still need wave 0
    asm volatile("" : "+v"(rq), "+v"(rqu), "+v"(bgv), "+v"(buv));
    const int tl = kg;  // 0: main, 1: tail
    const v4i a0 = red[tl][0][col], a1 = red[tl][1][col], u0 = red[tl][2][col], u1 = red[tl][3][col];
    int8_t fq = 0;
    if (en < p.N) {
      const uint16_t* sig = reinterpret_cast<const uint16_t*>(sig32);
      const int64_t tg = sat16(mulshift((int64_t)(a0.x + a1.x) + bgv, rq.x, rq.y));
      const int64_t tu = sat16(mulshift((int64_t)(u0.x + u1.x) + buv, rqu.x, rqu.y));
      if (p.g_out) p.g_out[en] = (int16_t)tg;
      if (p.u_out) p.u_out[en] = (int16_t)tu;
      // SiLU, the product's rounding shift and the quant in their exact 32-bit / double forms
      // (|tg|, |tu| < 2^15: silu16_fast's domain; |tu * sg| < 2^31)
      const int32_t sg = silu16_fast((int32_t)tg, mulshift_scale(p.silu_Mi, p.silu_Si), p.silu_sh, sig);
      const int32_t f = min(max(rshr32_any((int32_t)tu * sg, p.mul_sh), -32768), 32767);
      p.sg_out[en] = (int16_t)sg;
      p.f_out[en] = (int16_t)f;
      fq = (int8_t)mulshift_small_sat(f, mulshift_scale(p.fq_M, p.fq_S), -128.0, 127.0);
      p.fq_out[en] = fq;
    }
    fq16[tl][col] = fq;  // columns past N or past the group contribute nothing
  }
  __syncthreads();
  if (wave < 4) return;
  // down projection: the quantised FFN values of this workgroup's columns against every output column
  const v4i f4 = *reinterpret_cast<const v4i*>(fq16[0]);
  const v4i ft = *reinterpret_cast<const v4i*>(fq16[1]);
  int32_t* acc = p.wd_acc + (int64_t)(blockIdx.x % p.wd_R) * p.wd_N;
  auto dot16 = [](const v4i& f, const v4i& w, int32_t d) {
    d = __builtin_amdgcn_sdot4(f.x, w.x, d, false);
    d = __builtin_amdgcn_sdot4(f.y, w.y, d, false);
    d = __builtin_amdgcn_sdot4(f.z, w.z, d, false);
    return __builtin_amdgcn_sdot4(f.w, w.w, d, false);
  };
#pragma unroll
  for (int i = 0; i < WD_PF; ++i) {
    const int c = tid - 256 + 256 * i;
    const int32_t d = dot16(ft, wdt[i], dot16(f4, wdv[i], 0));
    if (c < p.wd_N && d != 0) atomic_add_dev(acc + c, d);
  }
  for (int c = tid - 256 + 256 * WD_PF; c < p.wd_N; c += 256) {
    int32_t d = dot16(f4, *reinterpret_cast<const v4i*>(p.wdp + ((int64_t)blockIdx.x * p.wd_N + c) * 16), 0);
    if (t0 >= 0) {
      const int8_t* tr = p.wdp + ((int64_t)(t0 >> 4) * p.wd_N + c) * 16 + (t0 & 15);
#pragma unroll
      for (int j = 0; j < GW; j += 4) d = __builtin_amdgcn_sdot4(reinterpret_cast<const int*>(fq16[1])[j >> 2],
                                                                 *reinterpret_cast<const int*>(tr + j), d, false);
    }
    if (d != 0) atomic_add_dev(acc + c, d);
  }
}

// ---------------------------------------------------------------------------------------
// norm_gemv: rmsnorm -> quant -> one linear with any epilogue (TPW 16-column tiles per
// workgroup, KS K-splits per tile)
// ---------------------------------------------------------------------------------------
struct NormGemvArgs {
  NormQuant pre;
  const int8_t* W;
  const int32_t* rq;
  const int32_t* bias;
  const int16_t* aux;
  void* out;
  int64_t Mi;
  int aux_shift, Si, sh, epilogue, out_i8;
  int M, N, K, KS, TPW;
  // decode chain (one row): with keys, the greedy step's first half -- keys[tile] = the best
  // (value, lowest index) key of the tile's columns below vocab, and the row recorded at
  // ring[*step] when *step < ring_cap
  uint64_t* keys;
  const int32_t* step;
  int16_t* ring;
  int64_t ring_ld;
  int ring_cap, vocab;
};

template <int MAXW>
__global__ __launch_bounds__(64 * MAXW) void norm_gemv_kernel(NormGemvArgs p) {
  kernarg_warm<sizeof(NormGemvArgs)>();
  extern __shared__ __attribute__((aligned(16))) int8_t dyn[];
  __shared__ v4i red[MAXW][64];
  __shared__ uint32_t sig32[129];
  const int lda = p.K + 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int col = lane & 15, kg = lane >> 4;
  const int t = wave % p.TPW, ks = wave / p.TPW;
  const int n = (blockIdx.x * p.TPW + t) * 16 + col;

  // the record slot of this decode launch (an earlier launch wrote it)
  int32_t stepv = ld4(rsrc(p.keys ? p.step : nullptr, 4), 0);
  const NormMap nm = norm_map(p.M);
  NormRegs nr;
  PreRows pq;
  if (p.pre.prequant)
    prerows_load(p.pre, p.M, pq);
  else
    norm_prefetch(p.pre, p.M, nm, nr);
  issue_fence();
  SigRegs sr;
  sig_prefetch(sr);
  issue_fence();
  const Rsrc wr = rsrc(p.W, (int64_t)p.N * p.K);
  WSlice<> ws;
  {
    int s0, s1;
    split_range((p.K + 63) >> 6, p.KS, ks, s0, s1);
    wslice_prefetch(ws, wr, n, p.K, kg, s0, s1);
  }
  issue_fence();
  const v2i rq = ld8(rsrc(p.rq, (int64_t)p.N * 8), n < p.N ? 8 * n : LD_OOB);
  const int32_t bias = ld4(rsrc(p.bias, (int64_t)p.N * 4), n < p.N ? 4 * n : LD_OOB);
  int32_t aux[4];
  {
    const bool use = p.epilogue == 1 || p.epilogue == 3;
    const Rsrc ar = rsrc(use ? p.aux : nullptr, (int64_t)p.M * p.N * 2);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * kg + r;
      aux[r] = ld2s(ar, (m < p.M && n < p.N) ? (uint32_t)(2 * ((int64_t)m * p.N + n)) : LD_OOB);
    }
  }
  issue_fence();

  if (p.pre.prequant)
    prerows_store(p.pre, p.M, pq, dyn, lda);
  else
    norm_quant_rows(p.pre, nr, p.M, nm, dyn, lda, blockIdx.x == 0);
  sig_store(sr, sig32);
  __syncthreads();
  v4i acc = wslice_mfma(ws, wr, dyn, lda, p.M, p.K);
  if (p.KS > 1) {
    red[wave][lane] = acc;
    __syncthreads();
    if (ks != 0) return;
    for (int j = 1; j < p.KS; ++j) v4_add(acc, red[t + j * p.TPW][lane]);
  }
  const uint16_t* sig = reinterpret_cast<const uint16_t*>(sig32);
  uint64_t key = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * kg + r;
    if (m >= p.M || n >= p.N) continue;
    const int64_t o = (int64_t)m * p.N + n;
    const int64_t v = mulshift((int64_t)acc[r] + bias, rq.x, rq.y);
    if (p.out_i8) {
      static_cast<int8_t*>(p.out)[o] = (int8_t)sat8(v);
      continue;
    }
    int64_t y = sat16(v);
    if (p.epilogue == 1) y = sat16(y + aux[r]);
    else if (p.epilogue == 2) y = silu16_lds(y, p.Mi, p.Si, p.sh, sig);
    else if (p.epilogue == 3) y = sat16(rshr(y * aux[r], p.aux_shift));
    static_cast<int16_t*>(p.out)[o] = (int16_t)y;
    if (p.keys && m == 0 && n < p.vocab) {
      key = amax_key((int)y, n);
      // the slot is needed from here on: the compiler may not make it uniform (and wait for its
      // load, before any other load is issued) at the kernel's start
      asm volatile("" : "+v"(stepv));
      if (stepv < p.ring_cap) p.ring[(int64_t)stepv * p.ring_ld + n] = (int16_t)y;
    }
  }
  if (p.keys) {
    // the tile's best key: lanes 0..15 hold its 16 columns (row 0)
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
      const uint32_t lo = __shfl_xor((uint32_t)key, off), hi = __shfl_xor((uint32_t)(key >> 32), off);
      const uint64_t o = ((uint64_t)hi << 32) | lo;
      key = o > key ? o : key;
    }
    const int tile = blockIdx.x * p.TPW + t;
    if (lane == 0 && tile * 16 < p.N) p.keys[tile] = key;
  }
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------

// Waves per workgroup are capped at 8 (512 threads, 256 VGPRs per lane) unless one split
// alone needs more (attn_in with D = 256): 16-wave workgroups leave 128 VGPRs per lane.
constexpr int FUSED_WAVES = 8;

// weight matrices are addressed with 32-bit buffer offsets
static bool w_ok(int64_t N, int64_t K) { return N * K < (1ll << 31); }

static int pick_ks(int64_t blocks, int per_split_waves, int steps, int max_waves) {
  const int target = 8 * current_cu_count();
  int ks = 1;
  while (per_split_waves * ks * 2 <= max_waves && blocks * per_split_waves * ks * 2 <= target && ks * 2 <= steps)
    ks *= 2;
  return ks;
}

}  // namespace llhip

using namespace llhip;

extern "C" int llhip_rmsnorm_quant(const llhip_norm_quant_desc* d, int64_t M, void* stream) {
  if (!d) return fail(-EINVAL, "rmsnorm_quant: null descriptor");
  NormQuant pr{};
  int rc = fill_pre(pr, *d);
  if (rc) return rc;
  if (M < 0 || M > INT32_MAX) return fail(-EINVAL, "rmsnorm_quant: bad row count");
  if (!d->hq_out && !d->h_out) return fail(-EINVAL, "rmsnorm_quant: no output");
  if (M == 0) return 0;
  hipLaunchKernelGGL(rmsnorm_quant_kernel, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream, pr);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

static int attn_in_args(const llhip_attn_in_desc* d, AttnInArgs& p, int& waves, size_t& lds, int min_threads) {
  if (!d) return fail(-EINVAL, "attn_in: null descriptor");
  int rc = fill_pre(p.pre, d->pre);
  if (rc) return rc;
  const int64_t M = d->M, H = d->H, Hkv = d->Hkv, D = d->D, K = d->pre.K;
  if (M < 1 || M > 16 || H < 1 || Hkv < 1 || H % Hkv || D < 16 || D > 256 || D % 16)
    return fail(-EINVAL, "attn_in: bad geometry (M <= 16, D multiple of 16 up to 256)");
  if (!d->pos_dev && !d->row_pos && (d->pos < 0 || d->pos + M > d->max_seq))
    return fail(-ERANGE, "positions %lld..%lld exceed max_seq=%lld", (long long)d->pos, (long long)(d->pos + M - 1),
                (long long)d->max_seq);
  for (int i = 0; i < 2; ++i)
    if (!u32_ok(d->quant_M[i]) || !shift_ok(d->quant_S[i]) ||
        (d->has_norm && (!u32_ok(d->nrm_eps[i]) || !u32_ok(d->nrm_C[i]) || !shift_ok(d->nrm_sh[i]))))
      return fail(-EINVAL, "attn_in: parameter out of range");
  for (int i = 0; i < 3; ++i) {
    p.W[i] = static_cast<const int8_t*>(d->W[i]);
    p.rq[i] = static_cast<const int32_t*>(d->rq[i]);
    p.bias[i] = static_cast<const int32_t*>(d->bias[i]);
    p.lin_out[i] = d->lin_out[i];
    if ((uintptr_t)p.W[i] % 16) return fail(-EINVAL, "attn_in: misaligned weights");
  }
  for (int i = 0; i < 2; ++i) {
    p.nrm_gamma[i] = static_cast<const int16_t*>(d->nrm_gamma[i]);
    p.nrm_out[i] = static_cast<int16_t*>(d->nrm_out[i]);
    p.nrm_eps[i] = d->nrm_eps[i];
    p.nrm_C[i] = d->nrm_C[i];
    p.nrm_sh[i] = d->nrm_sh[i];
    p.rope_out[i] = static_cast<int16_t*>(d->rope_out[i]);
    p.quant_out[i] = static_cast<int8_t*>(d->quant_out[i]);
    p.quant_M[i] = d->quant_M[i];
    p.quant_S[i] = d->quant_S[i];
  }
  p.cos_tab = static_cast<const int16_t*>(d->cos_tab);
  p.sin_tab = static_cast<const int16_t*>(d->sin_tab);
  p.pos_dev = static_cast<const int32_t*>(d->pos_dev);
  p.row_pos = static_cast<const int32_t*>(d->row_pos);
  p.slot_stride = d->slot_stride;
  if (p.row_pos && p.slot_stride < Hkv * d->max_seq * D) return fail(-EINVAL, "attn_in: cache slots overlap");
  p.kc = static_cast<int8_t*>(d->kc);
  p.vc = static_cast<int8_t*>(d->vc);
  p.max_seq = d->max_seq;
  p.M = (int)M;
  p.H = (int)H;
  p.Hkv = (int)Hkv;
  p.D = (int)D;
  p.K = (int)K;
  p.pos = (int)d->pos;
  p.has_norm = d->has_norm ? 1 : 0;
  const int tiles = (int)(D / 16);
  const int steps = (int)ceil_div(K, 64);
  if (!w_ok(H * D, K) || d->max_seq * D >= (1ll << 31)) return fail(-EINVAL, "attn_in: operand above 2 GiB");
  p.KS = pick_ks(H + 2 * Hkv, tiles, steps, tiles > FUSED_WAVES ? 16 : FUSED_WAVES);
  while (64 * tiles * p.KS < min_threads && p.KS < steps) ++p.KS;  // one row unit per thread
  lds = (size_t)((M * (K + 16) + 15) & ~15) + sizeof(int32_t) * (size_t)(M * D);
  if (lds > 48 * 1024) return fail(-EINVAL, "attn_in: M*K too large for the LDS staging");
  waves = tiles * p.KS;
  if (waves > 16 || 64 * waves < min_threads) return fail(-EINVAL, "attn_in: no workgroup shape fits");
  return 0;
}

template <bool RESID>
static int attn_in_launch(const AttnInArgs& p, int waves, size_t lds, void* stream) {
  const dim3 grid((unsigned)(p.H + 2 * p.Hkv)), block(64 * waves);
  if (waves <= FUSED_WAVES)
    hipLaunchKernelGGL((attn_in_kernel<FUSED_WAVES, RESID>), grid, block, lds, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL((attn_in_kernel<16, RESID>), grid, block, lds, (hipStream_t)stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

// The decode chain's attn_in with each head block over two workgroups (half of its 16-column
// tiles each, eight waves: more K splits per tile), when the head has no Q/K norm and its RoPE
// pairs stay within a half (D / 32 even).  Returns false when the shape does not allow it.
static bool attn_in_split_launch(AttnInArgs p, void* stream, int& rc) {
  constexpr int SPL = 2;
  const int tiles = p.D / 16 / SPL;
  if (p.has_norm || p.M != 1 || (p.D / 32) % SPL || tiles < 1 || FUSED_WAVES % tiles) return false;
  const int steps = (int)ceil_div(p.K, 64);
  const int ks = std::min(FUSED_WAVES / tiles, steps);
  if (64 * tiles * ks < p.K / 4 || (64 * tiles * ks) % (p.D / SPL)) return false;  // one row unit per thread
  p.KS = ks;
  const size_t lds = (size_t)((p.K + 16 + 15) & ~15) + sizeof(int32_t) * (size_t)p.D;
  if (ceil_div(steps, ks) <= 4)
    hipLaunchKernelGGL((attn_in_kernel<FUSED_WAVES, true, SPL, 4>), dim3((unsigned)((p.H + 2 * p.Hkv) * SPL)),
                       dim3(64 * tiles * ks), lds, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL((attn_in_kernel<FUSED_WAVES, true, SPL>), dim3((unsigned)((p.H + 2 * p.Hkv) * SPL)),
                       dim3(64 * tiles * ks), lds, (hipStream_t)stream, p);
  rc = hipGetLastError() == hipSuccess ? 0 : fail(-EIO, "dec_attn_in: launch failed");
  return true;
}

static int fill_resid(ResidArgs& ra, const llhip_resid_desc* r, const NormQuant& pre) {
  ra = ResidArgs{};
  ra.R = 1;
  if (!r || !r->acc) return 0;
  if (r->R < 1 || r->R > RESID_MAXR) return fail(-EINVAL, "decode chain: %lld accumulator rows (1..%d)",
                                                  (long long)r->R, RESID_MAXR);
  if (!r->rq || !r->aux) return fail(-EINVAL, "decode chain: the finished projection needs rq and the residual");
  if ((uintptr_t)r->acc % 16 || (uintptr_t)r->rq % 16 || (r->bias && (uintptr_t)r->bias % 16) ||
      (uintptr_t)r->aux % 8 || (r->x_out && (uintptr_t)r->x_out % 8))
    return fail(-EINVAL, "decode chain: misaligned operands");
  if (pre.K % 4) return fail(-EINVAL, "decode chain: row width must be a multiple of 4");
  ra.acc = static_cast<const int32_t*>(r->acc);
  ra.rq = static_cast<const int32_t*>(r->rq);
  ra.bias = static_cast<const int32_t*>(r->bias);
  ra.aux = static_cast<const int16_t*>(r->aux);
  ra.x_out = static_cast<int16_t*>(r->x_out);
  ra.R = (int)r->R;
  return 0;
}

static int check_zero(const void* zero, int64_t zero_n) {
  if (zero_n < 0 || zero_n > INT32_MAX || (zero_n && !zero) || (uintptr_t)zero % 16)
    return fail(-EINVAL, "decode chain: bad accumulator rows to clear");
  return 0;
}

extern "C" int llhip_attn_in(const llhip_attn_in_desc* d, void* stream) {
  AttnInArgs p{};
  int waves = 0;
  size_t lds = 0;
  const int rc = attn_in_args(d, p, waves, lds, 0);
  return rc ? rc : attn_in_launch<false>(p, waves, lds, stream);
}

extern "C" int llhip_dec_attn_in(const llhip_attn_in_desc* d, const llhip_resid_desc* r, void* zero, int64_t zero_n,
                                 void* stream) {
  if (!d) return fail(-EINVAL, "dec_attn_in: null descriptor");
  if (d->M != 1 || d->row_pos || d->pre.prequant) return fail(-EINVAL, "dec_attn_in: one row, one sequence");
  AttnInArgs p{};
  int waves = 0;
  size_t lds = 0;
  int rc = attn_in_args(d, p, waves, lds, (int)(d->pre.K / 4));
  if (!rc) rc = fill_resid(p.res, r, p.pre);
  if (!rc) rc = check_zero(zero, zero_n);
  if (rc) return rc;
  p.zero = static_cast<int32_t*>(zero);
  p.zero_n = (int)zero_n;
  if (attn_in_split_launch(p, stream, rc)) return rc;
  return attn_in_launch<true>(p, waves, lds, stream);
}

static int mlp_in_args(const llhip_mlp_in_desc* d, MlpInArgs& p, int min_threads) {
  if (!d) return fail(-EINVAL, "mlp_in: null descriptor");
  int rc = fill_pre(p.pre, d->pre);
  if (rc) return rc;
  const int64_t M = d->M, N = d->N, K = d->pre.K;
  if (M < 1 || M > 16 || N < 1) return fail(-EINVAL, "mlp_in: bad geometry (M <= 16)");
  if (!u32_ok(d->silu_Mi) || !shift_ok(d->silu_Si) || !shift_ok(d->silu_sh) || !shift_ok(d->mul_sh) ||
      !u32_ok(d->fq_M) || !shift_ok(d->fq_S))
    return fail(-EINVAL, "mlp_in: parameter out of range");
  if ((uintptr_t)d->Wg % 16 || (uintptr_t)d->Wu % 16) return fail(-EINVAL, "mlp_in: misaligned weights");
  p.Wg = static_cast<const int8_t*>(d->Wg);
  p.Wu = static_cast<const int8_t*>(d->Wu);
  p.rqg = static_cast<const int32_t*>(d->rqg);
  p.rqu = static_cast<const int32_t*>(d->rqu);
  p.bg = static_cast<const int32_t*>(d->bg);
  p.bu = static_cast<const int32_t*>(d->bu);
  p.g_out = static_cast<int16_t*>(d->g_out);
  p.u_out = static_cast<int16_t*>(d->u_out);
  p.sg_out = static_cast<int16_t*>(d->sg_out);
  p.f_out = static_cast<int16_t*>(d->f_out);
  p.fq_out = static_cast<int8_t*>(d->fq_out);
  p.silu_Mi = d->silu_Mi;
  p.silu_Si = (int)d->silu_Si;
  p.silu_sh = (int)d->silu_sh;
  p.mul_sh = (int)d->mul_sh;
  p.fq_M = d->fq_M;
  p.fq_S = (int)d->fq_S;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  const int tiles = (int)ceil_div(N, 16);
  if (!w_ok(N, K)) return fail(-EINVAL, "mlp_in: weights above 2 GiB");
  p.KS = pick_ks(tiles, 2, (int)ceil_div(K, 64), FUSED_WAVES);
  while (128 * p.KS < min_threads && 2 * p.KS < FUSED_WAVES) ++p.KS;  // one row unit per thread
  if (128 * p.KS < min_threads) return fail(-EINVAL, "mlp_in: no workgroup shape fits");
  const size_t lds = (size_t)(M * (K + 16));
  if (lds > 48 * 1024) return fail(-EINVAL, "mlp_in: M*K too large for the LDS staging");
  return 0;
}

extern "C" int llhip_mlp_in(const llhip_mlp_in_desc* d, void* stream) {
  MlpInArgs p{};
  const int rc = mlp_in_args(d, p, 0);
  if (rc) return rc;
  hipLaunchKernelGGL((mlp_in_kernel<FUSED_WAVES>), dim3((unsigned)ceil_div(p.N, 16)), dim3(128 * p.KS),
                     (size_t)(p.M * (p.K + 16)), (hipStream_t)stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_dec_mlp(const llhip_mlp_in_desc* d, const llhip_resid_desc* r, const void* wd_panel, void* wd_acc,
                             int64_t R, int64_t N_out, void* stream) {
  if (!d) return fail(-EINVAL, "dec_mlp: null descriptor");
  if (d->M != 1 || d->pre.prequant) return fail(-EINVAL, "dec_mlp: one row");
  MlpInArgs p{};
  int rc = mlp_in_args(d, p, (int)(d->pre.K / 4));
  if (!rc) rc = fill_resid(p.res, r, p.pre);
  if (rc) return rc;
  if (R < 1 || R > RESID_MAXR || N_out < 1 || N_out > INT32_MAX / 16 || !wd_panel || !wd_acc ||
      (uintptr_t)wd_panel % 16 || (uintptr_t)wd_acc % 16)
    return fail(-EINVAL, "dec_mlp: bad down-projection panel or accumulators");
  if (!w_ok(ceil_div(p.N, 16) * 16, N_out)) return fail(-EINVAL, "dec_mlp: down-projection panel above 2 GiB");
  p.wdp = static_cast<const int8_t*>(wd_panel);
  p.wd_acc = static_cast<int32_t*>(wd_acc);
  p.wd_R = (int)R;
  p.wd_N = (int)N_out;
  if (p.K > 4 * DM_THREADS / 2) return fail(-EINVAL, "dec_mlp: row width above %d", 4 * DM_THREADS / 2);
  // one workgroup per CU when the tiles past the CU count fit as one tail group per workgroup
  const int tiles = (int)ceil_div(p.N, 16), cus = current_cu_count();
  int W = tiles;
  p.tail_tiles = 0;
  p.tail_gw = 16;
  if (tiles > cus) {
    for (int gw = 4; gw <= 16; gw *= 2) {
      const int tt = tiles - cus;  // every group (u, i) lands on a workgroup below 8 * ceil(tt / 8) * (16 / gw)
      if (8 * ceil_div(tt, 8) * (16 / gw) <= cus) {
        W = cus;
        p.tail_tiles = tt;
        p.tail_gw = gw;
        break;
      }
    }
  }
  const dim3 grid((unsigned)W), block(DM_THREADS);
  const size_t lds = (size_t)(p.K + 16);
  if (p.tail_gw == 4)
    hipLaunchKernelGGL(dec_mlp_kernel<4>, grid, block, lds, (hipStream_t)stream, p);
  else if (p.tail_gw == 8)
    hipLaunchKernelGGL(dec_mlp_kernel<8>, grid, block, lds, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(dec_mlp_kernel<16>, grid, block, lds, (hipStream_t)stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

static int norm_linear_args(const llhip_norm_linear_desc* d, NormGemvArgs& p, int min_threads) {
  if (!d) return fail(-EINVAL, "norm_linear: null descriptor");
  int rc = fill_pre(p.pre, d->pre);
  if (rc) return rc;
  const int64_t M = d->M, N = d->N, K = d->pre.K;
  if (M < 1 || M > 16 || N < 1) return fail(-EINVAL, "norm_linear: bad geometry (M <= 16)");
  if (d->epilogue < 0 || d->epilogue > 3 || (d->out_i8 && d->epilogue != 0))
    return fail(-EINVAL, "norm_linear: bad epilogue");
  if ((d->epilogue == 1 || d->epilogue == 3) && !d->aux) return fail(-EINVAL, "norm_linear: epilogue needs aux");
  if (!shift_ok(d->aux_shift) || !shift_ok(d->silu_Si) || !shift_ok(d->silu_sh))
    return fail(-EINVAL, "norm_linear: shift out of [0,63]");
  if ((uintptr_t)d->W % 16) return fail(-EINVAL, "norm_linear: misaligned weights");
  p.W = static_cast<const int8_t*>(d->W);
  p.rq = static_cast<const int32_t*>(d->rq);
  p.bias = static_cast<const int32_t*>(d->bias);
  p.aux = static_cast<const int16_t*>(d->aux);
  p.out = d->out;
  p.Mi = d->silu_Mi;
  p.aux_shift = (int)d->aux_shift;
  p.Si = (int)d->silu_Si;
  p.sh = (int)d->silu_sh;
  p.epilogue = (int)d->epilogue;
  p.out_i8 = d->out_i8 ? 1 : 0;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  const int tiles = (int)ceil_div(N, 16);
  const int steps = (int)ceil_div(K, 64);
  if (!w_ok(N, K) || M * N * 2 >= (1ll << 31)) return fail(-EINVAL, "norm_linear: operand above 2 GiB");
  // wide outputs: several tiles per workgroup share one prologue, K split in two so every step of
  // a wave's slice is loaded at entry; narrow ones split K further
  p.TPW = tiles >= 4096 ? 4 : 1;
  p.KS = p.TPW == 1 ? pick_ks(tiles, 1, steps, FUSED_WAVES) : (steps > PF ? 2 : 1);
  while (64 * p.TPW * p.KS < min_threads && p.TPW * p.KS < FUSED_WAVES && p.KS < steps) ++p.KS;
  if (64 * p.TPW * p.KS < min_threads) return fail(-EINVAL, "norm_linear: no workgroup shape fits");
  const size_t lds = (size_t)(M * (K + 16));
  if (lds > 48 * 1024) return fail(-EINVAL, "norm_linear: M*K too large for the LDS staging");
  return 0;
}

static int norm_linear_launch(const NormGemvArgs& p, void* stream) {
  const int blocks = (int)ceil_div(ceil_div(p.N, 16), p.TPW);
  hipLaunchKernelGGL((norm_gemv_kernel<FUSED_WAVES>), dim3((unsigned)blocks), dim3(64 * p.TPW * p.KS),
                     (size_t)(p.M * (p.K + 16)), (hipStream_t)stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_norm_linear(const llhip_norm_linear_desc* d, void* stream) {
  NormGemvArgs p{};
  const int rc = norm_linear_args(d, p, 0);
  return rc ? rc : norm_linear_launch(p, stream);
}

// one row finished from partial sums, normalised and quantised by one workgroup (dec_finish)
__global__ __launch_bounds__(256) void dec_finish_kernel(NormQuant pre, ResidArgs res) {
  extern __shared__ __attribute__((aligned(16))) int8_t dyn[];
  __shared__ uint64_t red64[4];
  ResidRegs rr;
  resid_prefetch(pre, res, rr);
  resid_norm_quant(pre, res, rr, dyn, true, red64);
}

extern "C" int llhip_dec_finish(const llhip_norm_quant_desc* d, const llhip_resid_desc* r, void* stream) {
  if (!d) return fail(-EINVAL, "dec_finish: null descriptor");
  NormQuant pre{};
  int rc = fill_pre(pre, *d);
  if (rc) return rc;
  if (d->prequant || pre.K > 4 * 256) return fail(-EINVAL, "dec_finish: one row of at most 1024 values");
  ResidArgs res{};
  rc = fill_resid(res, r, pre);
  if (rc) return rc;
  hipLaunchKernelGGL(dec_finish_kernel, dim3(1), dim3(256), (size_t)(pre.K + 16), (hipStream_t)stream, pre, res);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_dec_head(const llhip_norm_linear_desc* d, int64_t vocab, void* keys, const int32_t* step,
                              int16_t* ring, int64_t ring_ld, int64_t ring_cap, void* stream) {
  if (!d) return fail(-EINVAL, "dec_head: null descriptor");
  if (d->M != 1) return fail(-EINVAL, "dec_head: one row");
  NormGemvArgs p{};
  const int rc = norm_linear_args(d, p, 0);
  if (rc) return rc;
  if (keys) {
    if (d->out_i8 || vocab < 1 || vocab > d->N || !step || (uintptr_t)keys % 8 || ring_cap < 0 ||
        (ring_cap && (!ring || ring_ld < vocab)))
      return fail(-EINVAL, "dec_head: bad greedy-step operands");
    p.keys = static_cast<uint64_t*>(keys);
    p.step = step;
    p.ring = ring;
    p.ring_ld = ring_ld;
    p.ring_cap = (int)std::min<int64_t>(ring_cap, INT32_MAX);
    p.vocab = (int)vocab;
  }
  return norm_linear_launch(p, stream);
}

// ---------------------------------------------------------------------------------------
// dec_logits: the decode head in ONE persistent launch -- every workgroup finishes the last down
// projection from its partial sums and normalises + quantises the row into LDS (workgroup 0 also
// stores the row's outputs), then streams its share of the lm_head's 16-column tiles (8 waves, each
// tile's weights loaded straight into registers one tile ahead) with the requant epilogue, the
// record row and the running (value, lowest index) key; each workgroup writes its best key through
// to memory and counts itself, and the last one takes the greedy step (token, record, position,
// step, next input row).  One workgroup per CU, so each waits for its stores once per launch.
// ---------------------------------------------------------------------------------------
constexpr int DL_THREADS = 512;
constexpr int DL_MAXG = 256;            // workgroups at most (one per CU)
constexpr int DL_KEYS = DL_MAXG + 1;    // key words of a launch: the keys, then the arrival counter

struct DecLogitsArgs {
  NormQuant pre;
  ResidArgs res;
  const int8_t* W;     // [N][K], or in tile order (PANEL): [ceil(N/16)][K/64][64 lanes][16]
  const int32_t* rq;   // [N][2]
  const int32_t* bias; // [N] or null
  int16_t* out;        // [N] logits, or null
  uint64_t* keys;      // [DL_KEYS]: one key per workgroup, then the arrival counter at DL_MAXG
  const int32_t* step;
  int16_t* ring;
  int64_t ring_ld;
  int32_t* token;
  int32_t* pos;
  int32_t* ring_tok;
  const int16_t* embed;
  int16_t* row;
  int N, K, vocab, ring_cap, dim;
};

template <int KS, bool PANEL>
__global__ __launch_bounds__(DL_THREADS) void dec_logits_kernel(DecLogitsArgs p) {
  kernarg_warm<sizeof(DecLogitsArgs)>();
  extern __shared__ __attribute__((aligned(16))) int8_t xq[];  // the quantised row, zeros to 64 KS bytes
  __shared__ uint64_t red64[8];
  __shared__ uint64_t best[8];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kg = lane >> 4;
  const int b = (int)blockIdx.x;
  const int tiles = (p.N + 15) / 16;
  const int tb0 = (int)((int64_t)b * tiles / gridDim.x), tb1 = (int)((int64_t)(b + 1) * tiles / gridDim.x);
  const Rsrc wr = rsrc(p.W, (int64_t)(PANEL ? 16 * tiles : p.N) * p.K), qr = rsrc(p.rq, (int64_t)p.N * 8),
             br = rsrc(p.bias, (int64_t)p.N * 4);
  const int nst = p.K / 64;
  // tile t's weights (lane (col, kg): bytes [64 s + 16 kg, +16) of column col for each K step s),
  // requant pair and bias; tiles past the workgroup's range read zeros
  auto load_tile = [&](int t, v4i* w, v2i& rq, int32_t& bias) {
    const int n = 16 * t + col;
    const bool in = t < tb1;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      // in tile order each load is 1 KiB in one piece; row-major, 16 pieces of 64 bytes
      const uint32_t off = PANEL ? (uint32_t)(((t * nst + s) * 64 + lane) * 16) : (uint32_t)(n * p.K + s * 64 + kg * 16);
      w[s] = ld16(wr, in && s < nst ? off : LD_OOB);
    }
    rq = ld8(qr, in && kg == 0 ? 8u * n : LD_OOB);
    bias = ld4(br, in && kg == 0 ? 4u * n : LD_OOB);
  };
  // three tiles' weights per wave in registers: two in flight while the third is multiplied
  v4i w0[KS], w1[KS], w2[KS];
  v2i q0{0, 0}, q1{0, 0}, q2{0, 0};
  int32_t b0 = 0, b1 = 0, b2 = 0;
  int t = tb0 + wave;
  load_tile(t, w0, q0, b0);  // requested before the row's finish (they do not depend on it)
  load_tile(t + 8, w1, q1, b1);
  // the finished, normalised, quantised row (golden.py:316-342, 124-137, 119-120)
  ResidRegs rr;
  resid_prefetch(p.pre, p.res, rr);
  for (int i = p.K + 4 * tid; i < 64 * KS; i += 4 * DL_THREADS) *reinterpret_cast<int32_t*>(xq + i) = 0;
  resid_norm_quant(p.pre, p.res, rr, xq, b == 0, red64);  // ends with a barrier
  const int32_t stepv = ld4(rsrc(p.step, 4), 0);
  uint64_t key = 0;
  auto tile = [&](int tt, const v4i* w, v2i rq, int32_t bias) {
    v4i acc = {0, 0, 0, 0};
    // the row is read from LDS for each tile (an offset the compiler cannot see through keeps the
    // reads in the loop): registers held for it would leave too few for three tiles of weights
    uint32_t xo = 16u * kg;
    __asm__ volatile("" : "+v"(xo));
#pragma unroll
    for (int s = 0; s < KS; ++s) {  // steps past K: zero weights times the zeroed tail of xq
      const v4i xa = *reinterpret_cast<const v4i*>(xq + s * 64 + xo);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, w[s], acc, 0, 0, 0);
    }
    if (lane < 16) {  // one input row: every output row equals row 0
      const int n = 16 * tt + lane;
      if (n < p.N) {
        const int16_t y = (int16_t)sat16(mulshift((int64_t)acc.x + bias, rq.x, rq.y));
        if (p.out) p.out[n] = y;
        if (n < p.vocab) {
          const uint64_t k = amax_key((int)y, n);
          key = k > key ? k : key;
          if (stepv < p.ring_cap) p.ring[(int64_t)stepv * p.ring_ld + n] = y;
        }
      }
    }
  };
  for (; t < tb1; t += 24) {
    load_tile(t + 16, w2, q2, b2);
    tile(t, w0, q0, b0);
    if (t + 8 >= tb1) break;
    load_tile(t + 24, w0, q0, b0);
    tile(t + 8, w1, q1, b1);
    if (t + 16 >= tb1) break;
    load_tile(t + 32, w1, q1, b1);
    tile(t + 16, w2, q2, b2);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)key, off), hi = __shfl_xor((uint32_t)(key >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    key = o > key ? o : key;
  }
  if (lane == 0) best[wave] = key;
  __syncthreads();
  if (tid == 0) {
    uint64_t k = best[0];
    for (int w = 1; w < 8; ++w) k = best[w] > k ? best[w] : k;
    // through to memory: the last workgroup reads it
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2i, k), rsrc(p.keys, DL_KEYS * 8), 8u * b, 0, 16);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the key landed
    uint32_t* cnt = reinterpret_cast<uint32_t*>(p.keys + DL_MAXG);
    last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1u;
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
  }
  __syncthreads();
  if (!last) return;
  // the greedy step (golden.py:376-377, record golden.py:411-414, next row golden.py:369-373)
  if (wave == 0) {
    const Rsrc kr = rsrc(p.keys, DL_KEYS * 8);
    uint64_t k = 0;
    for (int i = lane; i < (int)gridDim.x; i += 64) {
      const uint64_t v = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(kr, 8u * i, 0, 16));
      k = v > k ? v : k;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t lo = __shfl_xor((uint32_t)k, off), hi = __shfl_xor((uint32_t)(k >> 32), off);
      const uint64_t o = ((uint64_t)hi << 32) | lo;
      k = o > k ? o : k;
    }
    if (lane == 0) {
      // every column below vocab made a nonzero key; a zero maximum cannot occur
      const int32_t idx = k ? (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull)) : 0;
      last = idx;
      *p.token = idx;
      if (stepv < p.ring_cap) p.ring_tok[stepv] = idx;
      *p.pos = *p.pos + 1;
      *const_cast<int32_t*>(p.step) = stepv + 1;
    }
  }
  __syncthreads();
  const int16_t* src = p.embed + (int64_t)last * p.dim;
  for (int i = tid; i < p.dim; i += blockDim.x) p.row[i] = src[i];
}

extern "C" int llhip_dec_logits(const llhip_norm_linear_desc* d, const void* panel, const llhip_resid_desc* r,
                                int64_t vocab, void* keys,
                                int32_t* token, int32_t* pos, int32_t* step, int16_t* ring, int64_t ring_ld,
                                int32_t* ring_tokens, int64_t ring_cap, const int16_t* embed, int64_t dim, int16_t* row,
                                void* stream) {
  if (!d) return fail(-EINVAL, "dec_logits: null descriptor");
  DecLogitsArgs p{};
  int rc = fill_pre(p.pre, d->pre);
  if (rc) return rc;
  if (d->pre.prequant || d->M != 1 || d->epilogue != 0 || d->out_i8) return fail(-EINVAL, "dec_logits: one row, plain epilogue");
  rc = fill_resid(p.res, r, p.pre);
  if (rc) return rc;
  const int64_t N = d->N, K = d->pre.K;
  if (N < 16 || K % 64 || K > NORM_MAX_K || !w_ok(ceil_div(N, 16) * 16, K) || (uintptr_t)d->W % 16 ||
      (uintptr_t)panel % 16)
    return fail(-EINVAL, "dec_logits: lm_head geometry (K a multiple of 64, at most %d; W 16-byte aligned)", NORM_MAX_K);
  const int G = std::min(current_cu_count(), DL_MAXG);
  if (!keys || (uintptr_t)keys % 8 || vocab < 1 || vocab > N || !step || !token || !pos || ring_cap < 0 ||
      (ring_cap && (!ring || ring_ld < vocab || !ring_tokens)) || !embed || dim < 1 || dim > INT32_MAX || !row)
    return fail(-EINVAL, "dec_logits: bad greedy-step operands");
  p.W = static_cast<const int8_t*>(panel ? panel : d->W);
  p.rq = static_cast<const int32_t*>(d->rq);
  p.bias = static_cast<const int32_t*>(d->bias);
  p.out = static_cast<int16_t*>(d->out);
  p.keys = static_cast<uint64_t*>(keys);
  p.step = step;
  p.ring = ring;
  p.ring_ld = ring_ld;
  p.token = token;
  p.pos = pos;
  p.ring_tok = ring_tokens;
  p.embed = embed;
  p.row = row;
  p.N = (int)N;
  p.K = (int)K;
  p.vocab = (int)vocab;
  p.ring_cap = (int)std::min<int64_t>(ring_cap, INT32_MAX);
  p.dim = (int)dim;
  const hipStream_t st = (hipStream_t)stream;
  if (K <= 576)
    hipLaunchKernelGGL((panel ? dec_logits_kernel<9, true> : dec_logits_kernel<9, false>), dim3(G), dim3(DL_THREADS),
                       64 * 9, st, p);
  else if (K <= 896)
    hipLaunchKernelGGL((panel ? dec_logits_kernel<14, true> : dec_logits_kernel<14, false>), dim3(G), dim3(DL_THREADS),
                       64 * 14, st, p);
  else
    hipLaunchKernelGGL((panel ? dec_logits_kernel<16, true> : dec_logits_kernel<16, false>), dim3(G), dim3(DL_THREADS),
                       64 * 16, st, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

// The greedy step of a decode chain (golden.py:376-377 and the record of golden.py:411-414): the
// best of the tiles' keys is the first argmax; then token, record, position and step updates, and
// the next launch's input row = embed[token] (golden.py:369-373).
__global__ __launch_bounds__(1024) void dec_greedy_kernel(const uint64_t* __restrict__ keys, int nkeys, int32_t* token,
                                                          int32_t* pos, int32_t* step, int32_t* ring_tok, int ring_cap,
                                                          const int16_t* __restrict__ embed, int dim, int16_t* row) {
  __shared__ uint64_t best[16];
  __shared__ int32_t win;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t k = 0;
  constexpr int BATCH = 16;  // keys in flight per thread
  for (int base = tid; base < nkeys; base += BATCH * (int)blockDim.x) {
    uint64_t v[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int i = base + j * (int)blockDim.x;
      v[j] = i < nkeys ? keys[i] : 0ull;
    }
#pragma unroll
    for (int j = 0; j < BATCH; ++j) k = v[j] > k ? v[j] : k;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)k, off), hi = __shfl_xor((uint32_t)(k >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    k = o > k ? o : k;
  }
  if (lane == 0) best[wave] = k;
  __syncthreads();
  if (tid == 0) {
    uint64_t b = best[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = best[w] > b ? best[w] : b;
    // every tile with a column below vocab wrote a nonzero key; a zero maximum cannot occur
    const int32_t idx = b ? (int32_t)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull)) : 0;
    win = idx;
    *token = idx;
    const int32_t s = *step;
    if (s < ring_cap) ring_tok[s] = idx;
    *pos = *pos + 1;
    *step = s + 1;
  }
  __syncthreads();
  const int16_t* src = embed + (int64_t)win * dim;
  for (int i = tid; i < dim; i += blockDim.x) row[i] = src[i];
}

extern "C" int llhip_dec_greedy(const void* keys, int64_t nkeys, int32_t* token, int32_t* pos, int32_t* step,
                                int32_t* ring_tokens, int64_t ring_cap, const int16_t* embed, int64_t dim, int16_t* row,
                                void* stream) {
  if (!keys || nkeys < 1 || nkeys > INT32_MAX || !token || !pos || !step || ring_cap < 0 ||
      (ring_cap && !ring_tokens) || !embed || dim < 1 || dim > INT32_MAX || !row)
    return fail(-EINVAL, "dec_greedy: bad arguments");
  hipLaunchKernelGGL(dec_greedy_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream,
                     static_cast<const uint64_t*>(keys), (int)nkeys, token, pos, step, ring_tokens,
                     (int)std::min<int64_t>(ring_cap, INT32_MAX), embed, (int)dim, row);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int64_t llhip_dec_head_keys(int64_t N) { return ceil_div(N, 16); }

extern "C" int64_t llhip_dec_logits_keys(void) { return DL_KEYS; }

// one 16-byte piece per thread: piece i = (tile t, K step s, lane l = 16 kg + c)
__global__ __launch_bounds__(256) void dec_logits_panel_kernel(const int8_t* __restrict__ W, int N, int K,
                                                               int64_t pieces, v4i* __restrict__ panel) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pieces) return;
  const int nst = K / 64, l = (int)(i & 63);
  const int64_t ts = i >> 6;
  const int t = (int)(ts / nst), s = (int)(ts % nst);
  const int n = 16 * t + (l & 15);
  panel[i] = n < N ? *reinterpret_cast<const v4i*>(W + (int64_t)n * K + 64 * s + 16 * (l >> 4)) : v4i{0, 0, 0, 0};
}

extern "C" int llhip_dec_logits_panel(const void* W, int64_t N, int64_t K, void* panel, void* stream) {
  if (!W || !panel || N < 1 || K < 64 || K % 64 || !w_ok(ceil_div(N, 16) * 16, K) || (uintptr_t)W % 16 ||
      (uintptr_t)panel % 16)
    return fail(-EINVAL, "dec_logits_panel: bad operands (K a multiple of 64, 16-byte aligned)");
  const int64_t pieces = ceil_div(N, 16) * (K / 64) * 64;
  hipLaunchKernelGGL(dec_logits_panel_kernel, dim3((unsigned)ceil_div(pieces, 256)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const int8_t*>(W), (int)N, (int)K, pieces, static_cast<v4i*>(panel));
  LLHIP_LAUNCH_CHECK();
  return 0;
}
