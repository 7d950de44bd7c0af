// gemm engine of libllhip: out = epilogue(requant(A . W^T + bias)) with int8
// operands, exact int32 accumulation and the i64 requant of golden.py:316-342
// (NUMERICS.md "GEMM").
//
// Two kernels:
//  * linear_gemv: M <= 16 rows per z-block (decode GEMV, prefill chunks).  One workgroup
//    per 16-column tile; its waves split the K range and each computes a 16(M) x 16(N)
//    partial tile with v_mfma_i32_16x16x64_i8 (A rows beyond M are zeros supplied in
//    registers); the partials are summed in LDS.  W [N][K] row-major is streamed once
//    with 16-byte loads, four K steps in flight per wave.  Integer addition is
//    associative, so the split never changes a result.
//  * linear_tiled: M > 16.  128x256 (or 128x128) x 64 block tiles, four waves in 2x2,
//    each wave 64x128 (64x64) with v_mfma_i32_32x32x32_i8; A and W double-buffered in LDS.
//    Blocks are numbered XCD-major so the blocks that share a W panel run on one
//    XCD and share its L2.
#include <algorithm>
#include <type_traits>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {

typedef int v16i __attribute__((ext_vector_type(16)));

enum Epi : int { EPI_NONE = 0, EPI_RESADD = 1, EPI_SILU = 2, EPI_MUL = 3, EPI_ROPE = 4 };


struct LinearArgs {
  const int8_t* A;
  const int8_t* W;
  const int32_t* rq;
  const int32_t* bias;
  const int16_t* aux;
  void* out;
  int64_t lda, ldaux, ldo;
  int64_t Mi;
  int M, K, N;
  int aux_shift, Si, sh;
  int steps;  // ceil(K / 64)
  int cpb;    // linear_gemv: output columns per workgroup (16, or 8 / 4 to spread narrow outputs)
  int nfast;   // linear_mfma: tiles in N-fastest order (N-block l % nblk), else M-fastest
  int nblk;
  int mgroup;  // M-fastest order within groups of mgroup M-blocks (0: one group of all)
};

// M-block and N-block of logical tile l: N-block fastest (nfast), or M-block fastest within groups
// of mgroup M-blocks whose A rows fit an L2 together (the groups one after another), or M-block
// fastest over all of them
__device__ __forceinline__ void tile_mn(const LinearArgs& p, int mblocks, int l, int& mb, int& nb) {
  if (p.nfast) {
    mb = l / p.nblk;
    nb = l % p.nblk;
  } else if (p.mgroup && mblocks > p.mgroup) {
    const int gsz = p.mgroup * p.nblk, g = l / gsz, r = l % gsz;
    const int gm = min(p.mgroup, mblocks - g * p.mgroup);
    mb = g * p.mgroup + r % gm;
    nb = r / gm;
  } else {
    mb = l % mblocks;
    nb = l / mblocks;
  }
}

// requant + epilogue of one output element (golden.py:323-342)
template <int EPI, bool OUT8>
__device__ __forceinline__ void finish(const LinearArgs& p, int m, int n, int64_t acc) {
  if (p.bias) acc += p.bias[n];
  const int64_t Mn = p.rq[2 * n];
  const int Sn = p.rq[2 * n + 1];
  const int64_t r = mulshift(acc, Mn, Sn);
  if (OUT8) {
    static_cast<int8_t*>(p.out)[(int64_t)m * p.ldo + n] = (int8_t)sat8(r);
    return;
  }
  int64_t t = sat16(r);
  if (EPI == EPI_RESADD) {
    t = sat16(t + p.aux[(int64_t)m * p.ldaux + n]);
  } else if (EPI == EPI_SILU) {
    t = silu16(t, p.Mi, p.Si, p.sh);
  } else if (EPI == EPI_MUL) {
    t = sat16(rshr(wmul(t, p.aux[(int64_t)m * p.ldaux + n]), p.aux_shift));
  }
  static_cast<int16_t*>(p.out)[(int64_t)m * p.ldo + n] = (int16_t)t;
}

// 16 bytes of a K-contiguous row starting at k (zeros past K)
template <bool ALIGNED>
__device__ __forceinline__ v4i load16(const int8_t* row, int k, int K, bool valid) {
  if (ALIGNED) {
    if (valid && k < K) return *reinterpret_cast<const v4i*>(row + k);
    return v4i{0, 0, 0, 0};
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
    if (valid) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        int kk = k + i;
        uint32_t b = kk < K ? (uint8_t)row[kk] : 0u;
        w[i >> 2] |= b << (8 * (i & 3));
      }
    }
    return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

// ---------------------------------------------------------------------------------------
// M <= 16 (per z-block): one workgroup per 16-column tile, K split across its waves
// ---------------------------------------------------------------------------------------
// Wave w of the workgroup accumulates the K steps [w*spw, (w+1)*spw) of the tile with
// v_mfma_i32_16x16x64_i8; the per-wave 16x16 partial tiles are summed through LDS by wave 0,
// which applies the epilogue.  No workgroup depends on another, so the kernel needs no
// device-scope synchronisation (on the multi-XCD part those fences flush the XCD's L2).
constexpr int GEMV_MAX_WAVES = 16;

// epilogue operands of one lane's column n and rows m0 + 4*kg + r, loaded before the MFMAs
template <int EPI>
struct EpiOperands {
  int64_t rq_m;
  int rq_s;
  int32_t bias;
  int16_t aux[4];
};

template <int EPI, bool OUT8>
__device__ __forceinline__ void finish_pre(const LinearArgs& p, const EpiOperands<EPI>& e, int r, int m, int n,
                                           int64_t acc) {
  const int64_t v = mulshift(acc + e.bias, e.rq_m, e.rq_s);
  if (OUT8) {
    static_cast<int8_t*>(p.out)[(int64_t)m * p.ldo + n] = (int8_t)sat8(v);
    return;
  }
  int64_t t = sat16(v);
  if (EPI == EPI_RESADD) t = sat16(t + e.aux[r]);
  else if (EPI == EPI_SILU) t = silu16(t, p.Mi, p.Si, p.sh);
  else if (EPI == EPI_MUL) t = sat16(rshr(wmul(t, e.aux[r]), p.aux_shift));
  static_cast<int16_t*>(p.out)[(int64_t)m * p.ldo + n] = (int16_t)t;
}

constexpr int GEMV_PF = 8;  // K steps of W and A in flight per wave

template <int EPI, bool OUT8, bool ALIGNED>
__global__ __launch_bounds__(64 * GEMV_MAX_WAVES) void linear_gemv(LinearArgs p) {
  __shared__ v4i red[GEMV_MAX_WAVES - 1][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int col = lane & 15;
  const int kg = lane >> 4;
  const int tile = blockIdx.x;  // columns [tile * cpb, tile * cpb + cpb): lanes col >= cpb carry zero weights
  const int m0 = blockIdx.z * 16;
  const int n = tile * p.cpb + col;
  const bool nvalid = col < p.cpb && n < p.N;
  const int nn = nvalid ? n : 0;
  const bool avalid = m0 + col < p.M;
  const int8_t* wrow = p.W + (int64_t)nn * p.K;
  const int8_t* arow = p.A + (int64_t)(avalid ? m0 + col : 0) * p.lda;

  const int spw = (p.steps + nw - 1) / nw;
  const int s_begin = min(wave * spw, p.steps);
  const int s_end = min(s_begin + spw, p.steps);
  v4i acc = {0, 0, 0, 0};
  int s = s_begin;
  // first GEMV_PF steps: every load issued before the first MFMA
  {
    v4i b[GEMV_PF], a[GEMV_PF];
#pragma unroll
    for (int u = 0; u < GEMV_PF; ++u) {
      const int k = (s + u) * 64 + kg * 16;
      const bool ok = s + u < s_end;
      b[u] = ok ? load16<ALIGNED>(wrow, k, p.K, nvalid) : v4i{0, 0, 0, 0};
      a[u] = ok ? load16<ALIGNED>(arow, k, p.K, avalid) : v4i{0, 0, 0, 0};
    }
    EpiOperands<EPI> e{};
    if (wave == 0) {
      e.rq_m = p.rq[2 * nn];
      e.rq_s = p.rq[2 * nn + 1];
      e.bias = p.bias ? p.bias[nn] : 0;
      if (EPI == EPI_RESADD || EPI == EPI_MUL) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 4 * kg + r;
          e.aux[r] = m < p.M ? p.aux[(int64_t)m * p.ldaux + nn] : (int16_t)0;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < GEMV_PF; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
    s += GEMV_PF;
    constexpr int U = 4;
    for (; s < s_end; s += U) {
      v4i bb[U], aa[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = (s + u) * 64 + kg * 16;
        const bool ok = s + u < s_end;
        bb[u] = ok ? load16<ALIGNED>(wrow, k, p.K, nvalid) : v4i{0, 0, 0, 0};
        aa[u] = ok ? load16<ALIGNED>(arow, k, p.K, avalid) : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(aa[u], bb[u], acc, 0, 0, 0);
    }
    if (nw > 1) {
      if (wave > 0) red[wave - 1][lane] = acc;
      __syncthreads();
      if (wave > 0) return;
      for (int w = 0; w < nw - 1; ++w) {
        const v4i o = red[w][lane];
        acc.x += o.x;
        acc.y += o.y;
        acc.z += o.z;
        acc.w += o.w;
      }
    }
    // acc[r] = C[4*kg + r][col] of this 16x16 tile
    if (nvalid) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 4 * kg + r;
        if (m < p.M) finish_pre<EPI, OUT8>(p, e, r, m, n, acc[r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// M = 1 with few output columns (decode projections): VALU dot products, one wave per CPW
// columns, no LDS and no barrier
// ---------------------------------------------------------------------------------------
// With 16-column MFMA tiles an N = 896 projection has 56 workgroups, so a quarter of the CUs
// carry all of its weight traffic.  Here lane l of a wave works on column l / LPC of the wave's
// CPW = 64 / LPC columns and on the 16-byte K chunks l % LPC + i*LPC, with v_dot4_i32_i8; the
// LPC partial sums of a column are folded with lane shuffles and its first lane applies the
// epilogue.  Every load of a lane (up to G1_PF chunks of W and of A, and the epilogue operands)
// is issued at entry.
constexpr int G1_PF = 8;

template <int EPI, bool OUT8, int LPC>
__global__ __launch_bounds__(64) void linear_gemv1(LinearArgs p) {
  kernarg_warm<sizeof(LinearArgs)>();
  constexpr int CPW = 64 / LPC;
  const int lane = threadIdx.x;
  const int c = lane / LPC, j = lane % LPC;
  const int n = blockIdx.x * CPW + c;
  const int nch = p.K >> 4;
  const Rsrc wr = rsrc(p.W, (int64_t)p.N * p.K), ar = rsrc(p.A, p.K);
  const uint32_t row = (uint32_t)n * (uint32_t)p.K;  // columns n >= N read zeros
  v4i w[G1_PF], a[G1_PF];
#pragma unroll
  for (int u = 0; u < G1_PF; ++u) {
    const int ch = j + u * LPC;
    w[u] = ld16(wr, ch < nch ? row + 16 * ch : LD_OOB);
    a[u] = ld16(ar, ch < nch ? 16 * ch : LD_OOB);
  }
  issue_fence();
  const bool lead = j == 0 && n < p.N;
  const v2i rq = ld8(rsrc(p.rq, (int64_t)p.N * 8), lead ? 8 * n : LD_OOB);
  const int32_t bias = ld4(rsrc(p.bias, (int64_t)p.N * 4), lead ? 4 * n : LD_OOB);
  const int32_t aux =
      (EPI == EPI_RESADD || EPI == EPI_MUL) ? ld2s(rsrc(p.aux, (int64_t)p.N * 2), lead ? 2 * n : LD_OOB) : 0;
  issue_fence();
  int32_t acc = 0;
#pragma unroll
  for (int u = 0; u < G1_PF; ++u) {
    acc = __builtin_amdgcn_sdot4(w[u].x, a[u].x, acc, false);
    acc = __builtin_amdgcn_sdot4(w[u].y, a[u].y, acc, false);
    acc = __builtin_amdgcn_sdot4(w[u].z, a[u].z, acc, false);
    acc = __builtin_amdgcn_sdot4(w[u].w, a[u].w, acc, false);
  }
  for (int ch0 = G1_PF * LPC; ch0 < nch; ch0 += G1_PF * LPC) {
#pragma unroll
    for (int u = 0; u < G1_PF; ++u) {
      const int ch = ch0 + j + u * LPC;
      w[u] = ld16(wr, ch < nch ? row + 16 * ch : LD_OOB);
      a[u] = ld16(ar, ch < nch ? 16 * ch : LD_OOB);
    }
#pragma unroll
    for (int u = 0; u < G1_PF; ++u) {
      acc = __builtin_amdgcn_sdot4(w[u].x, a[u].x, acc, false);
      acc = __builtin_amdgcn_sdot4(w[u].y, a[u].y, acc, false);
      acc = __builtin_amdgcn_sdot4(w[u].z, a[u].z, acc, false);
      acc = __builtin_amdgcn_sdot4(w[u].w, a[u].w, acc, false);
    }
  }
  acc = group_sum_i32<LPC>(acc);
  if (!lead) return;
  const int64_t v = mulshift((int64_t)acc + bias, rq.x, rq.y);
  if (OUT8) {
    static_cast<int8_t*>(p.out)[n] = (int8_t)sat8(v);
    return;
  }
  int64_t t = sat16(v);
  if (EPI == EPI_RESADD) t = sat16(t + aux);
  else if (EPI == EPI_SILU) t = silu16(t, p.Mi, p.Si, p.sh);
  else if (EPI == EPI_MUL) t = sat16(rshr(wmul(t, aux), p.aux_shift));
  static_cast<int16_t*>(p.out)[n] = (int16_t)t;
}

// ---------------------------------------------------------------------------------------
// M > 16: LDS-tiled MFMA GEMM (K % 16 == 0)
// ---------------------------------------------------------------------------------------
// Block = 2 x 2 waves; a wave owns a (32*WM) x (32*WN) tile of v_mfma_i32_32x32x32_i8 blocks.
// Per 64-deep K tile the block stages A [BM][64] and W [BN][64] in LDS (rows padded to 80 B,
// conflict-free 16-byte reads), double-buffered: the global loads of tile k+1 are in flight while
// tile k feeds the MFMAs.  Epilogue: per output column the requant multiplier M_n, shift S_n and
// bias*M_n are loaded once, so (acc + bias) * M_n is one 32x32->64 multiply-add per element.
constexpr int TBK = 64;
constexpr int TLD = TBK + 16;  // LDS row stride in bytes (pad against bank conflicts)

template <int EPI, bool OUT8>
__device__ __forceinline__ void store_out(const LinearArgs& p, int m, int n, int64_t v, int16_t aux) {
  if (OUT8) {
    static_cast<int8_t*>(p.out)[(int64_t)m * p.ldo + n] = (int8_t)sat8(v);
    return;
  }
  int64_t t = sat16(v);
  if (EPI == EPI_RESADD) t = sat16(t + aux);
  else if (EPI == EPI_SILU) t = silu16(t, p.Mi, p.Si, p.sh);
  else if (EPI == EPI_MUL) t = sat16(rshr(wmul(t, aux), p.aux_shift));
  static_cast<int16_t*>(p.out)[(int64_t)m * p.ldo + n] = (int16_t)t;
}

template <int EPI, bool OUT8, int WM, int WN>
__global__ __launch_bounds__(256) void linear_tiled(LinearArgs p, int mblocks, int nblocks) {
  constexpr int BM = 64 * WM, BN = 64 * WN;
  constexpr int ACH = BM * 4 / 256, BCH = BN * 4 / 256;  // 16-byte chunks per thread per K tile
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * TLD];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * TLD];

  // XCD-major block numbering: hardware dispatches block b to XCD b % 8
  const int nb_total = mblocks * nblocks;
  const int b = blockIdx.x;
  int logical = b;
  if (nb_total % 8 == 0) logical = (b % 8) * (nb_total / 8) + b / 8;
  const int mb = logical % mblocks;
  const int nbk = logical / mblocks;
  const int m0 = mb * BM, n0 = nbk * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave & 1) * 32 * WM, wn = (wave >> 1) * 32 * WN;

  v4i ra[ACH], rb[BCH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 2, gk = k0 + (c & 3) * 16, gm = m0 + row;
      ra[i] = (gm < p.M && gk < p.K) ? *reinterpret_cast<const v4i*>(p.A + (int64_t)gm * p.lda + gk) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 2, gk = k0 + (c & 3) * 16, gn = n0 + row;
      rb[i] = (gn < p.N && gk < p.K) ? *reinterpret_cast<const v4i*>(p.W + (int64_t)gn * p.K + gk) : v4i{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<v4i*>(&As[buf][(c >> 2) * TLD + (c & 3) * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<v4i*>(&Bs[buf][(c >> 2) * TLD + (c & 3) * 16]) = rb[i];
    }
  };

  v16i acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v16i{};

  const int ktiles = (p.K + TBK - 1) / TBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) gload((kt + 1) * TBK);
#pragma unroll
    for (int ks = 0; ks < TBK; ks += 32) {
      v4i fa[WM], fb[WN];
      const int koff = ks + 16 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < WM; ++i)
        fa[i] = *reinterpret_cast<const v4i*>(&As[buf][(wm + 32 * i + (lane & 31)) * TLD + koff]);
#pragma unroll
      for (int j = 0; j < WN; ++j)
        fb[j] = *reinterpret_cast<const v4i*>(&Bs[buf][(wn + 32 * j + (lane & 31)) * TLD + koff]);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) sstore(buf ^ 1);
    __syncthreads();
  }

  // C layout of a 32x32 tile: lane l, element r -> row (r/4)*8 + (l/32)*4 + r%4, col l%32
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int n = n0 + wn + 32 * j + (lane & 31);
    if (n >= p.N) continue;
    const int32_t Mn = p.rq[2 * n];
    const int Sn = p.rq[2 * n + 1];
    const int64_t bM = (int64_t)(p.bias ? p.bias[n] : 0) * Mn;  // (acc + bias) * M = acc * M + bias * M
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 32 * i + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (m >= p.M) continue;
        const int64_t v = rshr((int64_t)acc[i][j][r] * Mn + bM, Sn);
        const int16_t aux = (EPI == EPI_RESADD || EPI == EPI_MUL) ? p.aux[(int64_t)m * p.ldaux + n] : (int16_t)0;
        store_out<EPI, OUT8>(p, m, n, v, aux);
      }
  }
}

// Requant of one accumulator, rshr((int64)acc * M + bias * M, S) (= golden.py's
// mulshift(acc + bias, M, S)), returned clamped to int32 (every later step saturates to 8 or 16
// bits, so the clamp changes no output).  Round-half-up is floor((v + 2^(S-1)) / 2^S), so with the
// constant bR = bias * M + 2^(S-1) folded in and 32 <= S <= 62 the result is the high word of
// acc * M + bR shifted right by S - 32: one v_mad_i64_i32 and one shift.  |acc| < 2^30 and
// |M|, |bias| <= 2^31 keep acc * M + bR below 2^63.
struct ColRq {
  int32_t M;
  int S;
  int64_t bR;  // bias * M + 2^(S-1) (bias * M when S = 0)
};

__device__ __forceinline__ ColRq make_colrq(int32_t M, int S, int32_t bias) {
  ColRq c;
  c.M = M;
  c.S = S;
  c.bR = (int64_t)bias * M + (S > 0 ? (int64_t)1 << (S - 1) : 0);
  // opaque to the optimiser (emits nothing): otherwise acc * M + bR is refactored into a
  // 64 x 32-bit product instead of one v_mad_i64_i32 per element
  __asm__ volatile("" : "+v"(c.bR));
  return c;
}

__device__ __forceinline__ bool colrq_fast(const ColRq& c) { return c.S >= 32 && c.S <= 62; }

// requant of one accumulator: rshr((acc + bias) * M, S) (golden.py:323-337).  FAST (S in [32, 62]):
// for K <= 2^16, |(acc + bias) * M| < 1.5 * 2^62, so adding the rounding bit before the shift cannot
// overflow and the high word shifted by S - 32 is the result.  Otherwise the reference's
// overflow-free rounding shift of the 64-bit product (bias * M recovered from bR, not kept per
// column).
template <bool FAST>
__device__ __forceinline__ int32_t requant_col(int32_t acc, const ColRq& c) {
  if (FAST) return (int32_t)(((int64_t)acc * (int64_t)c.M + c.bR) >> 32) >> (c.S - 32);
  const int64_t bM = c.bR - (c.S > 0 ? (int64_t)1 << (c.S - 1) : 0);
  const int64_t v = (int64_t)acc * (int64_t)c.M + bM;
  return (int32_t)clamp64(rshr(v, c.S), INT32_MIN, INT32_MAX);
}

__device__ __forceinline__ int32_t clamp32(int32_t v, int32_t lo, int32_t hi) { return min(max(v, lo), hi); }

// ---------------------------------------------------------------------------------------
// Large GEMM (M >= 128, K % 64 == 0): GM x GN block tile (256 x 256 with 8 waves, 128 x 128 or
// 64 x 128 with 4) over K tiles of KT bytes (128 where K allows it, else 64) in an NS-stage LDS ring
// fed by direct global->LDS loads (global_load_lds_dwordx4)
// ---------------------------------------------------------------------------------------
// Each wave instruction moves 64 x 16 B into 1 KiB of LDS: RPL = 1024 / KT rows of KT bytes.  Lane L
// writes slot L of that KiB (row L / (KT/16), slot L % (KT/16)) and fetches K chunk slot ^ swz(row),
// so a row's 16-byte chunks are stored XOR-permuted and the fragment reads of 16 consecutive rows at
// one K chunk fall into distinct LDS banks without padding.  With 128-byte K tiles every row's part
// of a load is a whole 128-byte line (8 rows per instruction): 16 rows x 64 B per instruction moved
// 16 TB/s from L2 to LDS, 8 rows x 128 B 21-30 TB/s (the contiguous-KiB rate), and the 2048 x 896 x
// 151936 GEMM went 441 -> 406 us.  The ring holds NS = 4 tiles of 64 bytes or 2 of 128.  The K loop
// reads the fragments of the next 32-byte K step while the MFMAs of this one run; once all of tile
// kt's fragments are in registers one barrier frees its stage for tile kt + NS and publishes tile
// kt + 1 (landed when at most the loads of tiles kt+2 .. kt+NS-1 are outstanding).  Rows past M/N
// read a clamped valid row (their outputs are discarded); K is a multiple of KT, so no chunk is
// partial.  Deeper rings (up to 12 stages in 144 KB, one workgroup per CU) measured slower on the
// prompt-sized GEMMs: their K loop is not bound by the number of tiles in flight.
constexpr int GSTAGES = 4;

// 16-byte K chunk c of row r sits in slot c ^ swz(r) (64-byte rows: lds_swz; 128-byte: stage_swz<128>).
// Both are periodic in r with period 32, so fragment blocks 32 rows apart share their slot pattern.
__device__ __forceinline__ int lds_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
template <int KT>
__device__ __forceinline__ int stage_swz(int r) {
  if constexpr (KT == 64)
    return lds_swz(r);
  else
    return ((r >> 1) ^ (r << 2)) & 7;
}
// ring depth: 4 tiles of 64 bytes; 2 tiles of 128 bytes (two workgroups per CU for the smaller
// tile shapes), or 3 for a launch of fewer workgroups than CUs, where each one is alone on its CU
// and the deeper ring keeps more of its loads in flight (512 x 896 x 896: 8.7 -> 7.5 us)
template <int KT>
constexpr int ring_stages() {
  return KT == 64 ? GSTAGES : 2;
}
template <int GM, int GN, int KT>
constexpr bool deep_ring_fits() {
  return KT == 128 && (GM + GN) * KT * 3 <= 160 * 1024;
}

template <int GM, int GN, int NW, int KT = 64, int NSTAGES = ring_stages<KT>()>
struct MfmaTile {
  static constexpr int NT = 64 * NW;
  static constexpr int NS = NSTAGES;
  static constexpr int STAGE_BYTES = (GM + GN) * KT;  // A + W of one K tile
  static constexpr int LDS_BYTES = NS * STAGE_BYTES;
  static constexpr int WROWS = GM / 2;                // wave tile: 2 x NW/2 waves
  static constexpr int WCOLS = 2 * GN / NW;
  static constexpr int WM = WROWS / 32, WN = WCOLS / 32;  // 32x32 MFMA tiles per wave
  static constexpr int RPL = 1024 / KT;                   // rows per 1 KiB load instruction
  static constexpr int CPR = KT / 16;                     // 16-byte chunks per row
  static constexpr int KSTEPS = KT / 32;                  // 32-byte MFMA K steps per K tile
  static constexpr int LA = GM / (RPL * NW);              // 1 KiB A loads per wave per stage
  static constexpr int LW = GN / (RPL * NW);              // 1 KiB W loads per wave per stage
  static constexpr int LOADS = LA + LW;
  // accumulators read from their AGPRs at the point of use (off: the compiler keeps the
  // accumulators of every tile shape here in VGPRs, two waves per SIMD fit 256 of them)
  static constexpr bool AREG = false;
  static_assert(KT == 64 || KT == 128, "K tile bytes");
  static_assert(WM >= 1 && WN >= 1 && LA >= 1 && LW >= 1 && LA * RPL * NW == GM && LW * RPL * NW == GN, "tile shape");
  static_assert(NS >= 2 && LOADS * (NS - 1) <= 63, "vmcnt counts at most 63 loads");
  static_assert(LA <= 4 && LW <= 4, "load source arrays");
};

// An accumulator element read from its AGPR where it is used.  Without it the compiler copies all
// accumulators of a large tile into VGPRs after the K loop (and spills); with AREG false the value
// is used as it is.
template <bool AREG>
__device__ __forceinline__ int32_t acc_at(int32_t a) {
  if constexpr (AREG) {
    int32_t v;
    __asm__ volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
  } else {
    return a;
  }
}

// s_waitcnt vmcnt(N) (bits 3:0 and 15:14 of the immediate), expcnt and lgkmcnt not waited for
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt values");
  constexpr int imm = (N & 15) | ((N >> 4) << 14) | 0x0F70;
  __builtin_amdgcn_s_waitcnt(imm);
}

// wait until at most n tiles of L loads each are outstanding (n wave-uniform, n <= MAXN)
template <int L, int MAXN>
__device__ __forceinline__ void wait_tiles(int n) {
  if constexpr (MAXN <= 0) {
    wait_vmcnt<0>();
  } else {
    if (n >= MAXN)
      wait_vmcnt<L * MAXN>();
    else
      wait_tiles<L, MAXN - 1>(n);
  }
}

__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// interleave the MFMAs of one K step with the DS reads of the next (scheduling hint only)
template <int NMFMA, int NREAD>
__device__ __forceinline__ void mfma_ds_interleave() {
#pragma unroll
  for (int q = 0; q < NREAD; ++q) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
  }
  if constexpr (NMFMA > NREAD) __builtin_amdgcn_sched_group_barrier(0x008, NMFMA - NREAD, 0);
}

// i8-output epilogue straight from the accumulators: requant, then a 4x4 byte transpose across
// each lane quad (the 32x32 C layout gives lane l rows (r/4)*8 + (l/32)*4 + r%4 of column l%32;
// afterwards lane 4q+t of a half-wave holds row (r/4)*8 + (l/32)*4 + t, columns 4q..4q+3) and one
// dword store per four outputs.
template <bool FAST, bool AREG, int WM, int WN>
__device__ __forceinline__ void store_i8_tile(const LinearArgs& p, const v16i (&acc)[WM][WN], const ColRq (&cq)[WN],
                                              int mrow0, int ncol0, bool full) {
  const int lane = threadIdx.x & 63;
  const int t = lane & 3;
  const uint32_t sel1 = (t & 1) ? 0x03070105u : 0x06020400u;  // pair swap: bytes [x1 d1 x3 d3] / [d0 x0 d2 x2]
  const uint32_t sel2 = (t & 2) ? 0x03020706u : 0x05040100u;  // half swap: [y2 y3 d2 d3] / [d0 d1 y0 y1]
  int8_t* out = static_cast<int8_t*>(p.out);
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int nq = ncol0 + 32 * j + 4 * ((lane & 31) >> 2);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        int32_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = clamp32(requant_col<FAST>(acc_at<AREG>(acc[i][j][4 * g + q]), cq[j]), -128, 127);
        const uint32_t d = __builtin_amdgcn_perm((uint32_t)v[1], (uint32_t)v[0], 0x0c0c0400u) |
                           __builtin_amdgcn_perm((uint32_t)v[3], (uint32_t)v[2], 0x04000c0cu);
        const uint32_t d1 = __builtin_amdgcn_perm((uint32_t)dpp_mov<DPP_QUAD_XOR1>((int)d), d, sel1);
        const uint32_t e = __builtin_amdgcn_perm((uint32_t)dpp_mov<DPP_QUAD_XOR2>((int)d1), d1, sel2);
        const int m = mrow0 + 32 * i + g * 8 + (lane >> 5) * 4 + t;
        int8_t* dst = out + (int64_t)m * p.ldo + nq;
        if (full) {
          *reinterpret_cast<uint32_t*>(dst) = e;
        } else if (m < p.M) {
#pragma unroll
          for (int b = 0; b < 4; ++b)
            if (nq + b < p.N) dst[b] = (int8_t)(e >> (8 * b));
        }
        // the exact 64-bit form one output group at a time (its temporaries would otherwise be
        // interleaved across groups and raise the kernel's register peak)
        if constexpr (!FAST) __builtin_amdgcn_sched_barrier(0);
      }
  }
}

// i16-output epilogue straight from the accumulators: requant + sat16 in the C layout, a 4x4
// transpose of 16-bit values across each lane quad (an exchange of dwords with lane ^ 2, then of
// halves with lane ^ 1), after which lane 4q+t of a half-wave holds row (r/4)*8 + (l/32)*4 + t,
// columns 4q..4q+3: the aux operand is read and the result written 8 bytes at a time.
template <int EPI, bool FAST, bool AREG, int WM, int WN>
__device__ __forceinline__ void store_i16_tile(const LinearArgs& p, const v16i (&acc)[WM][WN], const ColRq (&cq)[WN],
                                               int mrow0, int ncol0, bool full, const uint16_t* sig) {
  const int lane = threadIdx.x & 63;
  const int t = lane & 3;
  const bool lo2 = t < 2;
  const uint32_t selh = (t & 1) ? 0x03020706u : 0x05040100u;  // odd: [x.hi | own.hi], even: [own.lo | x.lo]
  int16_t* out = static_cast<int16_t*>(p.out);
  // aux of every output group loaded before the first store: a load after a store to a pointer
  // that may alias it would wait for the store, one memory round trip per group
  constexpr bool AUX = EPI == EPI_RESADD || EPI == EPI_MUL;
  v2i axr[AUX ? WM : 1][AUX ? WN : 1][4];
  if (AUX && full) {
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int nq = ncol0 + 32 * j + 4 * ((lane & 31) >> 2);
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = mrow0 + 32 * i + g * 8 + (lane >> 5) * 4 + t;
          axr[AUX ? i : 0][AUX ? j : 0][g] = *reinterpret_cast<const v2i*>(p.aux + (int64_t)m * p.ldaux + nq);
        }
    }
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int nq = ncol0 + 32 * j + 4 * ((lane & 31) >> 2);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        int32_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = clamp32(requant_col<FAST>(acc_at<AREG>(acc[i][j][4 * g + q]), cq[j]), -32768, 32767);
        // E[lane][row]: d0 = rows 0,1, d1 = rows 2,3 of this lane's column
        const uint32_t d0 = __builtin_amdgcn_perm((uint32_t)v[1], (uint32_t)v[0], 0x05040100u);
        const uint32_t d1 = __builtin_amdgcn_perm((uint32_t)v[3], (uint32_t)v[2], 0x05040100u);
        const uint32_t r = (uint32_t)dpp_mov<DPP_QUAD_XOR2>((int)(lo2 ? d1 : d0));
        const uint32_t a = lo2 ? d0 : r, b = lo2 ? r : d1;  // rows {0,1} or {2,3} of lanes t and t^2
        const uint32_t t0 = __builtin_amdgcn_perm((uint32_t)dpp_mov<DPP_QUAD_XOR1>((int)a), a, selh);
        const uint32_t t1 = __builtin_amdgcn_perm((uint32_t)dpp_mov<DPP_QUAD_XOR1>((int)b), b, selh);
        const int m = mrow0 + 32 * i + g * 8 + (lane >> 5) * 4 + t;
        int32_t o[4] = {lo16((int)t0), hi16((int)t0), lo16((int)t1), hi16((int)t1)};
        if (full) {
          if (AUX) {
            const v2i ax = axr[AUX ? i : 0][AUX ? j : 0][g];
            const int32_t av[4] = {lo16(ax.x), hi16(ax.x), lo16(ax.y), hi16(ax.y)};
#pragma unroll
            for (int e = 0; e < 4; ++e)
              o[e] = EPI == EPI_RESADD ? clamp32(o[e] + av[e], -32768, 32767)
                                       : (int32_t)sat16(rshr((int64_t)(o[e] * av[e]), p.aux_shift));
          } else if (EPI == EPI_SILU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = silu16_i16(o[e], (uint32_t)p.Mi, p.Si, p.sh, sig);
          }
          // streamed past the caches (non-temporal): nothing in this launch reads the output, and
          // kept out of L2 it leaves the A and W panels there (512 x 896 x 151936: 152.6 -> 135.9
          // us; the same for the i8 stores above: 119 -> 160 us, not kept)
          __builtin_nontemporal_store(v2i{pack16(o[0], o[1]), pack16(o[2], o[3])},
                                      reinterpret_cast<v2i*>(out + (int64_t)m * p.ldo + nq));
        } else if (m < p.M) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int n = nq + e;
            if (n >= p.N) break;
            int32_t x = o[e];
            if (EPI == EPI_RESADD || EPI == EPI_MUL) {
              const int32_t aux = p.aux[(int64_t)m * p.ldaux + n];
              x = EPI == EPI_RESADD ? clamp32(x + aux, -32768, 32767) : (int32_t)sat16(rshr((int64_t)(x * aux), p.aux_shift));
            } else if (EPI == EPI_SILU) {
              x = silu16_i16(x, (uint32_t)p.Mi, p.Si, p.sh, sig);
            }
            out[(int64_t)m * p.ldo + n] = (int16_t)x;
          }
        }
      }
  }
}

// ---------------------------------------------------------------------------------------
// RoPE epilogue of the q/k/v projections of a prompt chunk (llhip_linear_group_rope): the tile's
// requantised values go through LDS (the ring is free after the K loop of a one-tile workgroup),
// then every thread takes 8 rotation pairs of one row and head -- columns i0..i0+7 and 32+i0.. of
// the 64-column head -- and applies the rope_quant kernel's arithmetic (golden.py:141-158, 119-120)
// with 16-byte table loads and 16- and 8-byte stores; key tiles also write the quantised keys into
// the K cache, value tiles their i8 rows into the V cache (golden.py:344-351).  Positions and cache
// slots as the rope_quant kernel's.
// ---------------------------------------------------------------------------------------
struct RopeShared {
  const int16_t* cos_tab;
  const int16_t* sin_tab;
  const int32_t* pos_dev;
  const int32_t* row_pos;
  int64_t table_rows, max_seq, slot_stride, seq_rows;
  int pos;
};
// one problem's part: kind 1 rope + quant [+ K cache], kind 2 V cache
struct RopeSel {
  int kind, qS;
  int64_t qM;
  int16_t* y;
  int8_t* yq;
  int8_t* cache;
};

__device__ __forceinline__ v4i rope_pack16x8(const int32_t (&v)[8]) {
  return v4i{pack16(v[0], v[1]), pack16(v[2], v[3]), pack16(v[4], v[5]), pack16(v[6], v[7])};
}
__device__ __forceinline__ v2i rope_pack8x8(const int32_t (&v)[8]) {
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e >> 2] |= (uint32_t)(v[e] & 255) << (8 * (e & 3));
  return v2i{(int)w[0], (int)w[1]};
}

// row m's position and cache slot (as the rope_quant kernel's)
__device__ __forceinline__ void rope_position(const RopeShared& rs, int64_t m, int64_t& pm, int64_t& slot) {
  pm = rs.row_pos ? (int64_t)rs.row_pos[m] : rs.seq_rows ? (int64_t)rs.pos + m % rs.seq_rows
                                                           : (int64_t)(rs.pos_dev ? *rs.pos_dev : rs.pos) + m;
  slot = rs.row_pos ? m * rs.slot_stride : (rs.seq_rows ? m / rs.seq_rows * rs.slot_stride : 0);
}

template <int GM, int GN, int NT, bool FAST, int WM, int WN>
__device__ __forceinline__ void rope_tile_epilogue(const LinearArgs& p, const v16i (&acc)[WM][WN],
                                                   const ColRq (&cq)[WN], int m0, int n0, int wm, int wn, int8_t* ring,
                                                   const RopeShared& rs, const RopeSel& sel, bool out8) {
  int16_t* X = reinterpret_cast<int16_t*>(ring);  // [GM][GN] requantised (i8 outputs: already clamped to i8)
  const int tid = threadIdx.x, lane = tid & 63;
#pragma unroll
  for (int j = 0; j < WN; ++j)
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm + 32 * i + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), col = wn + 32 * j + (lane & 31);
        const int32_t v = requant_col<FAST>(acc[i][j][r], cq[j]);
        X[row * GN + col] = (int16_t)(out8 ? clamp32(v, -128, 127) : clamp32(v, -32768, 32767));
      }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  lds_barrier();
  if (sel.kind == 1) {
    // item = (row, head of the tile, 8-pair group): GM x GN/64 x 4
    const double sq = mulshift_scale(sel.qM, sel.qS);
    constexpr int ITEMS = GM * (GN / 64) * 4;
#pragma unroll
    for (int k = 0; k < (ITEMS + NT - 1) / NT; ++k) {
      const int t = tid + k * NT;
      if (t >= ITEMS) break;
      const int row = t / ((GN / 64) * 4), rem = t % ((GN / 64) * 4), hh = rem >> 2, i0 = (rem & 3) * 8;
      const int64_t m = m0 + row;
      const int n = n0 + 64 * hh;  // the head's first column
      if (m >= p.M || n >= p.N) continue;
      const int16_t* xr = X + row * GN + 64 * hh + i0;
      const v4i a8 = *reinterpret_cast<const v4i*>(xr), b8 = *reinterpret_cast<const v4i*>(xr + 32);
      int16_t* out = static_cast<int16_t*>(p.out) + m * p.ldo + n + i0;  // the linear's own output
      *reinterpret_cast<v4i*>(out) = a8;
      *reinterpret_cast<v4i*>(out + 32) = b8;
      int64_t pm, slot;
      rope_position(rs, m, pm, slot);
      if (pm < 0 || pm >= rs.table_rows) continue;  // as the rope_quant kernel: no rotated output
      const int64_t trow = pm * 32 + i0;
      const v4i c8 = *reinterpret_cast<const v4i*>(rs.cos_tab + trow), s8 = *reinterpret_cast<const v4i*>(rs.sin_tab + trow);
      int32_t y1[8], y2[8], q1[8], q2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int32_t c = (e & 1) ? hi16(c8[e >> 1]) : lo16(c8[e >> 1]), sn = (e & 1) ? hi16(s8[e >> 1]) : lo16(s8[e >> 1]);
        const int32_t a = (e & 1) ? hi16(a8[e >> 1]) : lo16(a8[e >> 1]), b = (e & 1) ? hi16(b8[e >> 1]) : lo16(b8[e >> 1]);
        y1[e] = (int32_t)sat16(rshr((int64_t)a * c - (int64_t)b * sn, 14));
        y2[e] = (int32_t)sat16(rshr((int64_t)b * c + (int64_t)a * sn, 14));
        q1[e] = mulshift_small_sat(y1[e], sq, -128.0, 127.0);
        q2[e] = mulshift_small_sat(y2[e], sq, -128.0, 127.0);
      }
      const int64_t o = m * p.N + n + i0;  // rope and quant outputs: [M][H*D]
      if (sel.y) {
        *reinterpret_cast<v4i*>(sel.y + o) = rope_pack16x8(y1);
        *reinterpret_cast<v4i*>(sel.y + o + 32) = rope_pack16x8(y2);
      }
      const v2i w1 = rope_pack8x8(q1), w2 = rope_pack8x8(q2);
      *reinterpret_cast<v2i*>(sel.yq + o) = w1;
      *reinterpret_cast<v2i*>(sel.yq + o + 32) = w2;
      if (sel.cache && pm < rs.max_seq) {
        const int64_t dst = slot + ((int64_t)(n / 64) * rs.max_seq + pm) * 64 + i0;
        *reinterpret_cast<v2i*>(sel.cache + dst) = w1;
        *reinterpret_cast<v2i*>(sel.cache + dst + 32) = w2;
      }
    }
  } else {
    // value tile: item = (row, 16 columns); the i8 output and the V cache row
    for (int t = tid; t < GM * (GN / 16); t += NT) {
      const int row = t / (GN / 16), c0 = (t % (GN / 16)) * 16;
      const int64_t m = m0 + row;
      const int n = n0 + c0;
      if (m >= p.M || n >= p.N) continue;
      const int16_t* xr = X + row * GN + c0;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 16; ++e) w[e >> 2] |= (uint32_t)(xr[e] & 255) << (8 * (e & 3));
      const v4i v16 = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      *reinterpret_cast<v4i*>(static_cast<int8_t*>(p.out) + m * p.ldo + n) = v16;
      int64_t pm, slot;
      rope_position(rs, m, pm, slot);
      if (sel.cache && pm >= 0 && pm < rs.table_rows && pm < rs.max_seq)
        *reinterpret_cast<v4i*>(sel.cache + slot + ((int64_t)(n / 64) * rs.max_seq + pm) * 64 + (n % 64)) = v16;
    }
  }
}

// Output tiles l = l0, l0 + lstep, ... < lend (logical index l to M- and N-block by tile_mn), one
// after another.  The first stages of the next tile are issued as soon as the
// K loop of this one has finished reading the ring, so their memory latency passes during this
// tile's epilogue (which works from registers only).  The K-loop waits stay correct with the
// epilogue's stores in flight: vector loads complete in order, so at most n tiles' loads
// outstanding still means every earlier stage has landed.
// Split-K (part != NULL, one tile per workgroup): workgroup (tile, z = blockIdx.y) accumulates K
// tiles [z*kps, z*kps + kps) and stores its int32 partial tile into plane z of part
// [splits][M][N]; linear_splitk_finish sums the planes (integer addition: any split gives the same
// sum) and applies the epilogue.
template <int EPI, bool OUT8, int GM, int GN, int NW, int KT, int NS_>
__device__ __forceinline__ void mfma_tiles(const LinearArgs& p, int mblocks, int l0, int lstep, int lend, int kps,
                                           int32_t* part, const RopeShared* rs = nullptr, RopeSel rsel = RopeSel{}) {
  using T = MfmaTile<GM, GN, NW, KT, NS_>;
  constexpr int NS = T::NS;
  extern __shared__ __attribute__((aligned(1024))) int8_t ring[];  // [NS][A GM x KT | W GN x KT]
  if (l0 >= lend) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave & 1) * T::WROWS, wn = (wave >> 1) * T::WCOLS;

  // this lane's source rows for the LA A and LW W load instructions of a stage
  const int8_t* asrc[4];  // fixed sizes (see wait_vmcnt)
  const int8_t* wsrc[4];
  const int kbase = (int)blockIdx.y * kps * KT;  // first K byte of this split
  auto sources = [&](int l) {
    int mbi, nbi;
    tile_mn(p, mblocks, l, mbi, nbi);
    const int m0 = mbi * GM, n0 = nbi * GN;
    const int rl = lane / T::CPR, slot = lane % T::CPR;
#pragma unroll
    for (int i = 0; i < T::LA; ++i) {
      const int r = (wave * T::LA + i) * T::RPL + rl;
      const int gm = min(m0 + r, p.M - 1);
      asrc[i] = p.A + (int64_t)gm * p.lda + kbase + ((slot ^ stage_swz<KT>(r)) * 16);
    }
#pragma unroll
    for (int i = 0; i < T::LW; ++i) {
      const int r = (wave * T::LW + i) * T::RPL + rl;
      const int gn = min(n0 + r, p.N - 1);
      wsrc[i] = p.W + (int64_t)gn * p.K + kbase + ((slot ^ stage_swz<KT>(r)) * 16);
    }
  };
  auto issue = [&](int kt) {
    int8_t* st = ring + (kt % NS) * T::STAGE_BYTES;
    const int k0 = kt * KT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // explicitly typed operands (see wait_vmcnt)
      if (i < T::LA) {
        const int8_t* src = asrc[i] + k0;
        int8_t* dst = st + (wave * T::LA + i) * 1024;
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
      }
      if (i < T::LW) {
        const int8_t* src = wsrc[i] + k0;
        int8_t* dst = st + GM * KT + (wave * T::LW + i) * 1024;
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
      }
    }
  };
  // LDS offsets of this lane's fragments of block 0 for each 32-byte K step of a tile (block i / j
  // adds 32 * KT * i / j: the slot pattern repeats every 32 rows)
  int aoff[T::KSTEPS], woff[T::KSTEPS];
#pragma unroll
  for (int ks = 0; ks < T::KSTEPS; ++ks) {
    const int c = ks * 2 + (lane >> 5);  // 16-byte K chunk of this lane's fragment
    const int ra = wm + (lane & 31), rw = wn + (lane & 31);
    aoff[ks] = ra * KT + ((c ^ stage_swz<KT>(ra)) << 4);
    woff[ks] = GM * KT + rw * KT + ((c ^ stage_swz<KT>(rw)) << 4);
  }
  // SiLU table for the silu epilogue, staged in LDS (visible after the main loop's barriers)
  __shared__ uint32_t sig32[EPI == EPI_SILU ? 129 : 1];
  if (EPI == EPI_SILU && tid < 129) sig32[tid] = reinterpret_cast<const uint32_t*>(kSig)[tid];
  const uint16_t* sig16 = reinterpret_cast<const uint16_t*>(sig32);
  const int ktiles = min(kps, p.K / KT - (int)blockIdx.y * kps);
  sources(l0);
  for (int s0 = 0; s0 < NS; ++s0)
    if (s0 < ktiles) issue(s0);
  for (int l = l0;;) {
    int mbi, nbi;
    tile_mn(p, mblocks, l, mbi, nbi);
    const int m0 = mbi * GM, n0 = nbi * GN;
    // epilogue column parameters, loaded while the first K tiles stream in
    ColRq cq[T::WN];
#pragma unroll
    for (int j = 0; j < T::WN; ++j) {
      const int n = min(n0 + wn + 32 * j + (lane & 31), p.N - 1);
      cq[j] = make_colrq(p.rq[2 * n], p.rq[2 * n + 1], p.bias ? p.bias[n] : 0);  // (acc+bias)*M = acc*M + bias*M
    }

    v16i acc[T::WM][T::WN];
    // K tile 0 landed: the loads of the tiles issued after it may be outstanding
    wait_tiles<T::LOADS, NS - 1>(min(ktiles, NS) - 1);
    lds_barrier();
    v4i fa[2][T::WM], fb[2][T::WN];
    auto frags = [&](const int8_t* st, int ks, int buf) {
#pragma unroll
      for (int i = 0; i < T::WM; ++i) fa[buf][i] = *reinterpret_cast<const v4i*>(st + aoff[ks] + 32 * KT * i);
#pragma unroll
      for (int j = 0; j < T::WN; ++j) fb[buf][j] = *reinterpret_cast<const v4i*>(st + woff[ks] + 32 * KT * j);
    };
    // the MFMAs of one K step (the first of a tile's first K tile starts the accumulators at zero)
    auto mfmas = [&](int buf, bool zero) {
#pragma unroll
      for (int i = 0; i < T::WM; ++i)
#pragma unroll
        for (int j = 0; j < T::WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[buf][i], fb[buf][j], zero ? v16i{} : acc[i][j], 0, 0, 0);
      mfma_ds_interleave<T::WM * T::WN, T::WM + T::WN>();
    };
    frags(ring, 0, 0);
    // K tile kt: step s runs on fragment buffer s & 1 while step s+1's are read; after its last
    // reads (lgkmcnt(0)) and the barrier, stage kt % NS takes tile kt + NS and tile kt+1's first
    // fragments are read during the last step (after the last tile they come from a stale stage
    // and are never used)
    auto ktile = [&](int kt, auto first) {
      const int8_t* st = ring + (kt % NS) * T::STAGE_BYTES;
#pragma unroll
      for (int s = 0; s + 1 < T::KSTEPS; ++s) {
        frags(st, s + 1, (s + 1) & 1);
        mfmas(s & 1, decltype(first)::value && s == 0);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      wait_tiles<T::LOADS, NS - 1>(min(ktiles, kt + NS) - kt - 2);
      lds_barrier();
      if (kt + NS < ktiles) issue(kt + NS);
      frags(ring + ((kt + 1) % NS) * T::STAGE_BYTES, 0, T::KSTEPS & 1);
      mfmas((T::KSTEPS - 1) & 1, false);
    };
    ktile(0, std::true_type{});
    for (int kt = 1; kt < ktiles; ++kt) ktile(kt, std::false_type{});
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stale fragment reads have returned
    // the next tile's first stages, once every wave is done with the ring
    const int ln = l + lstep;
    if (ln < lend) {
      lds_barrier();
      sources(ln);
      for (int s0 = 0; s0 < NS; ++s0)
        if (s0 < ktiles) issue(s0);
    }

    if (part) {
      // C layout of a 32x32 tile: lane l, element r -> row (r/4)*8 + (l/32)*4 + r%4, col l%32; each
      // element store of the wave writes 2 rows x 128 contiguous bytes
      int32_t* plane = part + (int64_t)blockIdx.y * p.M * p.N;
#pragma unroll
      for (int j = 0; j < T::WN; ++j) {
        const int n = n0 + wn + 32 * j + (lane & 31);
#pragma unroll
        for (int i = 0; i < T::WM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm + 32 * i + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (m < p.M && n < p.N) plane[(int64_t)m * p.N + n] = acc_at<T::AREG>(acc[i][j][r]);
          }
      }
      if (ln >= lend) return;
      l = ln;
      continue;
    }

    // one wave-uniform choice of the requant form
    bool col_fast = true;
#pragma unroll
    for (int j = 0; j < T::WN; ++j) col_fast = col_fast && colrq_fast(cq[j]);
    const bool fast = __all(col_fast);

    if constexpr (EPI == EPI_ROPE) {  // one tile per workgroup: the ring is free (its reads returned above)
      lds_barrier();
      if (fast)
        rope_tile_epilogue<GM, GN, T::NT, true>(p, acc, cq, m0, n0, wm, wn, ring, *rs, rsel, OUT8);
      else
        rope_tile_epilogue<GM, GN, T::NT, false>(p, acc, cq, m0, n0, wm, wn, ring, *rs, rsel, OUT8);
      return;
    }

    if constexpr (OUT8) {
      const bool full = m0 + GM <= p.M && n0 + GN <= p.N && p.ldo % 4 == 0 && (uintptr_t)p.out % 4 == 0;
      if (fast)
        store_i8_tile<true, T::AREG>(p, acc, cq, m0 + wm, n0 + wn, full);
      else
        store_i8_tile<false, T::AREG>(p, acc, cq, m0 + wm, n0 + wn, full);
    } else {
      // i16 output (with the aux-reading epilogues) from registers as well
      const bool full = m0 + GM <= p.M && n0 + GN <= p.N && p.ldo % 4 == 0 && (uintptr_t)p.out % 8 == 0 &&
                        ((EPI != EPI_RESADD && EPI != EPI_MUL) || (p.ldaux % 4 == 0 && (uintptr_t)p.aux % 8 == 0));
      if (fast)
        store_i16_tile<EPI, true, T::AREG>(p, acc, cq, m0 + wm, n0 + wn, full, sig16);
      else
        store_i16_tile<EPI, false, T::AREG>(p, acc, cq, m0 + wm, n0 + wn, full, sig16);
    }
    if (ln >= lend) return;
    l = ln;
  }
}

// The grid is padded to a multiple of 8 and workgroup b runs on XCD b % 8, which takes a
// contiguous range of tiles (M fastest): the M-blocks that share a W panel share that XCD's L2.
// Persistent form (persist != 0, no split): the grid is a multiple of 8 workgroups, at most one
// per CU; XCD x takes the contiguous tile range [x * per, (x + 1) * per), per = ceil(tiles / 8),
// and its gridDim.x / 8 workgroups step through it together, so the ones running at any time still
// share W panels in that XCD's L2.
template <int EPI, bool OUT8, int GM, int GN, int NW, int KT, int NS>
__global__ __launch_bounds__(64 * NW) void linear_mfma(LinearArgs p, int mblocks, int nblocks, int kps, int32_t* part,
                                                       int persist) {
  const int b = blockIdx.x;
  const int tiles = mblocks * nblocks;
  if (persist) {
    const int per = (tiles + 7) / 8, x = b % 8, lo = x * per;
    mfma_tiles<EPI, OUT8, GM, GN, NW, KT, NS>(p, mblocks, lo + b / 8, (int)gridDim.x / 8, min(lo + per, tiles), kps, part);
    return;
  }
  const int logical = (b % 8) * (int)(gridDim.x / 8) + b / 8;
  mfma_tiles<EPI, OUT8, GM, GN, NW, KT, NS>(p, mblocks, logical, 1, min(logical + 1, tiles), kps, part);
}

// Several linears of one input in one launch (the q, k, v projections of a prompt chunk): the
// N-blocks of problem q are nb0[q] .. nb0[q+1]-1 of one grid; epilogue none, i8 or i16 output.
constexpr int GROUP_MAX = 4;
struct LinearGroup {
  int count;
  int nb0[GROUP_MAX + 1];
  const int8_t* W[GROUP_MAX];
  const int32_t* rq[GROUP_MAX];
  const int32_t* bias[GROUP_MAX];
  void* out[GROUP_MAX];
  int64_t ldo[GROUP_MAX];
  int N[GROUP_MAX];
  int out8[GROUP_MAX];
  // the RoPE epilogue (linear_mfma_group<..., true>): per problem, and shared
  RopeSel rope[GROUP_MAX];
  RopeShared rs;
};

template <int GM, int GN, int NW, int KT, int NS, bool ROPE = false>
__global__ __launch_bounds__(64 * NW) void linear_mfma_group(LinearArgs p, LinearGroup g, int mblocks) {
  const int b = blockIdx.x;
  const int logical = (b % 8) * (int)(gridDim.x / 8) + b / 8;
  if (logical >= mblocks * g.nb0[g.count]) return;
  const int mb = logical % mblocks;
  int nbk = logical / mblocks, q = 0;
  while (q + 1 < g.count && nbk >= g.nb0[q + 1]) ++q;
  LinearArgs pp = p;
  pp.W = g.W[q];
  pp.rq = g.rq[q];
  pp.bias = g.bias[q];
  pp.out = g.out[q];
  pp.ldo = g.ldo[q];
  pp.N = g.N[q];
  nbk -= g.nb0[q];
  const int l = nbk * mblocks + mb;
  if constexpr (ROPE) {
    // the problem's epilogue fields picked with a wave-uniform select (no indexed kernel argument)
    RopeSel sel = g.rope[0];
#pragma unroll
    for (int i = 1; i < GROUP_MAX; ++i)
      if (q == i) sel = g.rope[i];
    if (g.out8[q])
      mfma_tiles<EPI_ROPE, true, GM, GN, NW, KT, NS>(pp, mblocks, l, 1, l + 1, p.K / KT, nullptr, &g.rs, sel);
    else
      mfma_tiles<EPI_ROPE, false, GM, GN, NW, KT, NS>(pp, mblocks, l, 1, l + 1, p.K / KT, nullptr, &g.rs, sel);
    return;
  }
  if (g.out8[q])
    mfma_tiles<EPI_NONE, true, GM, GN, NW, KT, NS>(pp, mblocks, l, 1, l + 1, p.K / KT, nullptr);
  else
    mfma_tiles<EPI_NONE, false, GM, GN, NW, KT, NS>(pp, mblocks, l, 1, l + 1, p.K / KT, nullptr);
}

// ---------------------------------------------------------------------------------------
// gate + up of an MLP over many rows in one launch (golden.py:316-342 with the silu and mul
// epilogues, then quant golden.py:119-120): every 64x128 tile streams the gate and the up weight
// panels through one LDS ring against the same A rows, keeps both accumulators, and writes
// sg = silu16(requant16(A.Wg^T + bg)), f = sat16(rshr(requant16(A.Wu^T + bu) * sg, mul_sh)) and
// fq = quant(f) -- the values of the gate linear, the up linear and the quant run one by one.
// ---------------------------------------------------------------------------------------
struct DualArgs {
  const int8_t* Wu;
  const int32_t* rqu;
  const int32_t* bu;
  int16_t* sg;
  int16_t* f;
  int8_t* fq;
  int64_t ld;  // row stride of the three outputs (elements)
  int64_t fqM;
  int fqS, mul_sh;
};

// Eight waves: waves 0-3 accumulate the gate tile, waves 4-7 the up tile of the same 64xGN
// outputs (GN 128 or 64) from the same LDS stages (each wave the MFMA work of a 4-wave single
// GEMM tile, two waves per SIMD); the up waves pass their requantised values to the gate waves through LDS for the
// epilogue.  Stage loads: gate waves 1 A + 2 Wg instructions, up waves 2 Wu instructions.
template <int KT, int NS, int GN = 128>
__global__ __launch_bounds__(512) void linear_mfma_dual(LinearArgs p, DualArgs d, int mblocks, int nblocks) {
  constexpr int GM = 64;
  constexpr int RPL = 1024 / KT, CPR = KT / 16, KSTEPS = KT / 32;
  constexpr int LA = GM / (RPL * 4), LW = GN / (RPL * 4);  // 1 KiB loads per wave of one group
  constexpr int STAGE = (GM + 2 * GN) * KT;
  constexpr int WN = GN / 64;  // 32x32 tiles per wave along N (one along M)
  static_assert(LA >= 1 && LW >= 1 && (LA + LW) * (NS - 1) <= 63 && LA <= 4 && LW <= 4, "dual tile loads");
  // [NS][A | Wg | Wu]; after the k loop it holds the requantised gate and up tiles and the SiLU table
  // (80 KB: 4 stages of 64-byte or 2 of 128-byte K tiles, so two workgroups share a CU)
  extern __shared__ __attribute__((aligned(1024))) int8_t ring[];
  const int b = blockIdx.x;
  const int logical = (b % 8) * (int)(gridDim.x / 8) + b / 8;
  if (logical >= mblocks * nblocks) return;
  int mb, nbk;
  tile_mn(p, mblocks, logical, mb, nbk);  // M-block fastest, in groups when A exceeds an L2
  const int m0 = mb * GM, n0 = nbk * GN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool upw = wave >= 4;  // wave-uniform role: waves 0-3 gate (and the A loads), 4-7 up
  const int wq = wave & 3;
  const int wm = (wq & 1) * 32, wn = (wq >> 1) * (GN / 2);
  const int8_t* Wsrc = upw ? d.Wu : p.W;

  const int8_t* asrc[LA];
  const int8_t* wsrc[LW];
  {
    const int rl = lane / CPR, slot = lane % CPR;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int r = (wq * LA + i) * RPL + rl;
      asrc[i] = p.A + (int64_t)min(m0 + r, p.M - 1) * p.lda + ((slot ^ stage_swz<KT>(r)) * 16);
    }
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      const int r = (wq * LW + i) * RPL + rl;
      wsrc[i] = Wsrc + (int64_t)min(n0 + r, p.N - 1) * p.K + ((slot ^ stage_swz<KT>(r)) * 16);
    }
  }
  const int wbase = (upw ? GM + GN : GM) * KT;  // this wave group's W panel in a stage
  auto issue = [&](int kt) {
    int8_t* st = ring + (kt % NS) * STAGE;
    const int k0 = kt * KT;
    if (!upw) {
#pragma unroll
      for (int i = 0; i < LA; ++i) {
        const int8_t* src = asrc[i] + k0;
        int8_t* dst = st + (wq * LA + i) * 1024;
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      const int8_t* src = wsrc[i] + k0;
      int8_t* dst = st + wbase + (wq * LW + i) * 1024;
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
  };
  // vmcnt waits by wave group: gate waves issue LA + LW loads per stage, up waves LW
  auto wait_n = [&](int n) {
    if (upw)
      wait_tiles<LW, NS - 1>(n);
    else
      wait_tiles<LA + LW, NS - 1>(n);
  };
  // fragment offsets of block 0 per 32-byte K step (block j adds 32 * KT * j)
  int aoff[KSTEPS], woff[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    const int c = ks * 2 + (lane >> 5);
    const int ra = wm + (lane & 31), rw = wn + (lane & 31);
    aoff[ks] = ra * KT + ((c ^ stage_swz<KT>(ra)) << 4);
    woff[ks] = wbase + rw * KT + ((c ^ stage_swz<KT>(rw)) << 4);
  }
  const int32_t* rqp = upw ? d.rqu : p.rq;
  const int32_t* bp = upw ? d.bu : p.bias;
  ColRq cq[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int n = min(n0 + wn + 32 * j + (lane & 31), p.N - 1);
    cq[j] = make_colrq(rqp[2 * n], rqp[2 * n + 1], bp ? bp[n] : 0);
  }
  v16i acc[WN];

  // the K loop of mfma_tiles: tile kt's last fragments read, then one barrier frees its stage for
  // tile kt + NS and publishes tile kt + 1
  const int ktiles = p.K / KT;
  for (int s0 = 0; s0 < NS; ++s0)
    if (s0 < ktiles) issue(s0);
  wait_n(min(ktiles, NS) - 1);
  lds_barrier();
  v4i fa[2], fb[2][WN];
  auto frags = [&](const int8_t* st, int ks, int buf) {
    fa[buf] = *reinterpret_cast<const v4i*>(st + aoff[ks]);
#pragma unroll
    for (int j = 0; j < WN; ++j) fb[buf][j] = *reinterpret_cast<const v4i*>(st + woff[ks] + 32 * KT * j);
  };
  auto mfmas = [&](int buf, bool zero) {
#pragma unroll
    for (int j = 0; j < WN; ++j)
      acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[buf], fb[buf][j], zero ? v16i{} : acc[j], 0, 0, 0);
    mfma_ds_interleave<WN, 1 + WN>();
  };
  frags(ring, 0, 0);
  auto ktile = [&](int kt, auto first) {
    const int8_t* st = ring + (kt % NS) * STAGE;
#pragma unroll
    for (int s = 0; s + 1 < KSTEPS; ++s) {
      frags(st, s + 1, (s + 1) & 1);
      mfmas(s & 1, decltype(first)::value && s == 0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    wait_n(min(ktiles, kt + NS) - kt - 2);
    lds_barrier();
    if (kt + NS < ktiles) issue(kt + NS);
    frags(ring + ((kt + 1) % NS) * STAGE, 0, KSTEPS & 1);
    mfmas((KSTEPS - 1) & 1, false);
  };
  ktile(0, std::true_type{});
  for (int kt = 1; kt < ktiles; ++kt) ktile(kt, std::false_type{});
  __syncthreads();  // every wave's fragment reads have returned; no stage load is outstanding
  // Epilogue over all eight waves: each wave stores its requantised accumulators (gate or up, i16)
  // into the ring, then every thread finishes four adjacent columns of one row at a time from the
  // two tiles -- SiLU of the gate, the product with the up value, the quant -- and stores them as
  // 8-, 8- and 4-byte words.
  int16_t* gbuf = reinterpret_cast<int16_t*>(ring);  // [GM][GN] requantised gate
  int16_t* ubuf = gbuf + GM * GN;                      // [GM][GN] requantised up
  uint32_t* sig32 = reinterpret_cast<uint32_t*>(ubuf + GM * GN);
  if (tid < 129) sig32[tid] = reinterpret_cast<const uint32_t*>(kSig)[tid];
  const uint16_t* sig16 = reinterpret_cast<const uint16_t*>(sig32);
  {
    bool col_fast = true;
#pragma unroll
    for (int j = 0; j < WN; ++j) col_fast = col_fast && colrq_fast(cq[j]);
    int16_t* mine = upw ? ubuf : gbuf;
    // C layout of a 32x32 tile: lane l, element r -> row (r/4)*8 + (l/32)*4 + r%4, column l%32
    auto put = [&](auto fast) {
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ml = wm + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), nl = wn + 32 * j + (lane & 31);
          mine[ml * GN + nl] = (int16_t)clamp32(requant_col<decltype(fast)::value>(acc[j][r], cq[j]), -32768, 32767);
        }
    };
    if (__all(col_fast))
      put(std::true_type{});
    else
      put(std::false_type{});
  }
  __syncthreads();
  const double smul = mulshift_scale(p.Mi, p.Si), fqs = mulshift_scale(d.fqM, d.fqS);
  const bool vec = d.ld % 4 == 0 && (uintptr_t)d.sg % 8 == 0 && (uintptr_t)d.f % 8 == 0 && (uintptr_t)d.fq % 4 == 0;
  const bool keep_sg = d.sg != nullptr, keep_f = d.f != nullptr;  // NULL: that intermediate is not written
  constexpr int QPR = GN / 4;  // column quads per row
  for (int q = tid; q < GM * QPR; q += 512) {
    const int ml = q / QPR, nl = (q % QPR) * 4, m = m0 + ml, n = n0 + nl;
    if (m >= p.M) break;  // rows ascend with q
    const v2i gq = *reinterpret_cast<const v2i*>(gbuf + ml * GN + nl);
    const v2i uq = *reinterpret_cast<const v2i*>(ubuf + ml * GN + nl);
    const int32_t g4[4] = {lo16(gq.x), hi16(gq.x), lo16(gq.y), hi16(gq.y)};
    const int32_t u4[4] = {lo16(uq.x), hi16(uq.x), lo16(uq.y), hi16(uq.y)};
    int32_t sg[4], f[4], fq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sg[e] = silu16_fast(g4[e], smul, p.sh, sig16);
      f[e] = min(max(rshr32_any(u4[e] * sg[e], d.mul_sh), -32768), 32767);  // |u * sg| <= 2^30
      fq[e] = mulshift_small_sat(f[e], fqs, -128.0, 127.0);
    }
    const int64_t o = (int64_t)m * d.ld + n;
    if (vec && n + 4 <= p.N) {
      if (keep_sg) *reinterpret_cast<v2i*>(d.sg + o) = v2i{pack16(sg[0], sg[1]), pack16(sg[2], sg[3])};
      if (keep_f) *reinterpret_cast<v2i*>(d.f + o) = v2i{pack16(f[0], f[1]), pack16(f[2], f[3])};
      *reinterpret_cast<uint32_t*>(d.fq + o) = (uint32_t)(fq[0] & 255) | (uint32_t)(fq[1] & 255) << 8 |
                                               (uint32_t)(fq[2] & 255) << 16 | (uint32_t)(fq[3] & 255) << 24;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < p.N) {
          if (keep_sg) d.sg[o + e] = (int16_t)sg[e];
          if (keep_f) d.f[o + e] = (int16_t)f[e];
          d.fq[o + e] = (int8_t)fq[e];
        }
    }
  }
}

// sum of the split-K planes + bias, requant and epilogue; four columns per thread
// (every operand of a quad -- all planes, the requant pairs, bias, aux -- is requested before any is
// used: the stores of one quad may not be followed by its next loads in a dependent chain)
template <int EPI, bool OUT8>
__global__ __launch_bounds__(256) void linear_splitk_finish(LinearArgs p, const int32_t* part, int splits) {
  constexpr int MAXS = 8;  // launch_mfma splits K at most 8 ways
  const int64_t plane = (int64_t)p.M * p.N;
  const int64_t quads = plane / 4;
  const Rsrc prs = rsrc(part, (int64_t)splits * plane * 4);
  const Rsrc qr = rsrc(p.rq, (int64_t)p.N * 8), br = rsrc(p.bias, (int64_t)p.N * 4);
  constexpr bool AUX = EPI == EPI_RESADD || EPI == EPI_MUL;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < quads; q += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = 4 * q;
    const int m = (int)(e / p.N), n = (int)(e % p.N);  // N % 4 == 0: the quad stays in one row
    v4i pl[MAXS];
#pragma unroll
    for (int z = 0; z < MAXS; ++z) pl[z] = ld16(prs, z < splits ? (uint32_t)((z * plane + e) * 4) : LD_OOB);
    const v4i rq0 = ld16(qr, (uint32_t)(8 * n)), rq1 = ld16(qr, (uint32_t)(8 * n + 16));
    const v4i bi = ld16(br, (uint32_t)(4 * n));
    v2i ax = v2i{0, 0};
    if constexpr (AUX && !OUT8)
      ax = ld8(rsrc(p.aux + (int64_t)m * p.ldaux, (int64_t)p.N * 2), (uint32_t)(2 * n));
    v4i a = pl[0];
#pragma unroll
    for (int z = 1; z < MAXS; ++z) {  // planes past splits read zeros
      a.x += pl[z].x;
      a.y += pl[z].y;
      a.z += pl[z].z;
      a.w += pl[z].w;
    }
    const int32_t acc[4] = {a.x, a.y, a.z, a.w}, bias[4] = {bi.x, bi.y, bi.z, bi.w};
    const int32_t Mv[4] = {rq0.x, rq0.z, rq1.x, rq1.z}, Sv[4] = {rq0.y, rq0.w, rq1.y, rq1.w};
    const int32_t aux[4] = {lo16(ax.x), hi16(ax.x), lo16(ax.y), hi16(ax.y)};
    int32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t r = mulshift((int64_t)acc[j] + bias[j], (int64_t)Mv[j], Sv[j]);  // bias reads zeros when absent
      if (OUT8) {
        o[j] = (int32_t)sat8(r);
        continue;
      }
      int64_t t = sat16(r);
      if (EPI == EPI_RESADD) {
        t = sat16(t + aux[j]);
      } else if (EPI == EPI_SILU) {
        t = silu16(t, p.Mi, p.Si, p.sh);
      } else if (EPI == EPI_MUL) {
        t = sat16(rshr(wmul(t, aux[j]), p.aux_shift));
      }
      o[j] = (int32_t)t;
    }
    if (OUT8) {
      const uint32_t w = (uint32_t)(uint8_t)o[0] | ((uint32_t)(uint8_t)o[1] << 8) | ((uint32_t)(uint8_t)o[2] << 16) |
                         ((uint32_t)(uint8_t)o[3] << 24);
      *reinterpret_cast<uint32_t*>(static_cast<int8_t*>(p.out) + (int64_t)m * p.ldo + n) = w;
    } else {
      *reinterpret_cast<v2i*>(static_cast<int16_t*>(p.out) + (int64_t)m * p.ldo + n) =
          v2i{pack16(o[0], o[1]), pack16(o[2], o[3])};
    }
  }
}

// The split-K sum of a resadd linear and the RMSNorm + quant of its output rows in one launch
// (golden.py:316-342, then 124-137 + 119-120, as linear_splitk_finish followed by
// rmsnorm_quant_kernel): one 256-thread workgroup per row, thread t finishing columns 8t..8t+7 --
// planes summed, bias, requant, sat16, + aux, sat16 -- and writing them to the linear's output, then
// normalising and quantising them from registers once the row's sum of squares is reduced.
// N % 8 == 0, N <= NORM_MAX_K.
__device__ __forceinline__ void v4_acc(v4i& a, const v4i& b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

constexpr int FINISH_MAX_SPLITS = 8;  // launch_mfma splits K at most 8 ways

// One row per workgroup, 8 columns per thread.  Every operand is requested at entry (all planes'
// partial sums, requant pairs, bias, residual, gamma: 21 loads per thread, none waiting for another),
// then the sums, requant + resadd, the row's sum of squares, RMSNorm and quant.
__global__ __launch_bounds__(256) void splitk_finish_norm_kernel(LinearArgs p, const int32_t* part, int splits,
                                                                 NormQuant pr) {
  constexpr int NCH = NORM_MAX_K / 8 / 256 + 1;
  static_assert(NCH == 1, "one 8-column chunk per thread");
  __shared__ uint64_t red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nch = p.N >> 3;
  const int64_t plane = (int64_t)p.M * p.N;
  const int c = tid;
  const bool in = c < nch;
  const int64_t e = (int64_t)m * p.N + 8 * c;
  const Rsrc prs = rsrc(part, (int64_t)splits * plane * 4);
  v4i a[2 * FINISH_MAX_SPLITS];
#pragma unroll
  for (int z = 0; z < FINISH_MAX_SPLITS; ++z) {
    const uint32_t off = (in && z < splits) ? (uint32_t)((z * plane + e) * 4) : LD_OOB;
    a[2 * z] = ld16(prs, off);
    a[2 * z + 1] = ld16(prs, off == LD_OOB ? LD_OOB : off + 16);
  }
  const Rsrc qr = rsrc(p.rq, (int64_t)p.N * 8), br = rsrc(p.bias, (int64_t)p.N * 4);
  v4i rq[4], bi[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) rq[j] = ld16(qr, in ? (uint32_t)(64 * c + 16 * j) : LD_OOB);
#pragma unroll
  for (int j = 0; j < 2; ++j) bi[j] = ld16(br, in ? (uint32_t)(32 * c + 16 * j) : LD_OOB);
  const v4i ax = ld16(rsrc(p.aux + (int64_t)m * p.ldaux, (int64_t)p.N * 2), in ? (uint32_t)(16 * c) : LD_OOB);
  v4i g[NCH];
  g[0] = ld16(rsrc(pr.gamma, (int64_t)p.N * 2), in ? (uint32_t)(16 * c) : LD_OOB);
  v4i x[NCH];
  x[0] = v4i{0, 0, 0, 0};
  uint64_t ss = 0;
  if (in) {
    v4i a0 = a[0], a1 = a[1];
#pragma unroll
    for (int z = 1; z < FINISH_MAX_SPLITS; ++z) {  // planes past splits read zeros
      v4_acc(a0, a[2 * z]);
      v4_acc(a1, a[2 * z + 1]);
    }
    const int32_t acc[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const int32_t bias[8] = {bi[0].x, bi[0].y, bi[0].z, bi[0].w, bi[1].x, bi[1].y, bi[1].z, bi[1].w};
    const int32_t rqv[16] = {rq[0].x, rq[0].y, rq[0].z, rq[0].w, rq[1].x, rq[1].y, rq[1].z, rq[1].w,
                             rq[2].x, rq[2].y, rq[2].z, rq[2].w, rq[3].x, rq[3].y, rq[3].z, rq[3].w};
    const int32_t aux[8] = {lo16(ax.x), hi16(ax.x), lo16(ax.y), hi16(ax.y), lo16(ax.z), hi16(ax.z), lo16(ax.w), hi16(ax.w)};
    int32_t t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t v = (int64_t)acc[j] + bias[j];  // bias reads zeros when absent
      const int64_t r = sat16(mulshift(v, (int64_t)rqv[2 * j], rqv[2 * j + 1]));
      t[j] = (int32_t)sat16(r + aux[j]);
      ss += (uint32_t)(t[j] * t[j]);
    }
    x[0] = v4i{pack16(t[0], t[1]), pack16(t[2], t[3]), pack16(t[4], t[5]), pack16(t[6], t[7])};
    *reinterpret_cast<v4i*>(static_cast<int16_t*>(p.out) + (int64_t)m * p.ldo + 8 * c) = x[0];
  }
  ss = wave_sum_u64(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const uint32_t inv = rms_inv(red[0] + red[1] + red[2] + red[3], pr.eps_t, pr.C);
  const double sy = rms_scale(inv, pr.sh_post), sq = mulshift_scale(pr.Mq, pr.Sq);  // exact forms
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
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
    if (pr.hq_out) *reinterpret_cast<v2i*>(pr.hq_out + (int64_t)m * pr.K + 8 * c) = v2i{(int)qw[0], (int)qw[1]};
  }
}

// ---------------------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------------------
// One MFMA GEMM launch with GM x GN tiles of KT-byte K tiles.  Too few output tiles for the CUs
// (narrow projections of a prompt): split K into ranges of at least 256 bytes whose int32 partial
// tiles fit the workspace, then sum them.  The split count maximises (K-loop time saved) -
// (partial-plane traffic + the finishing launch), with measured costs: ~0.5 us (128x128) or ~0.4 us
// (64x128, also used for 64x64) per 64 bytes of K of a workgroup, ~5 us for the finishing launch and
// ~4 TB/s for the planes.  For 64x64 tiles the model's choice was checked directly: the prefill's
// 512 x 4864 x 896 down projection split 5 ways (the model's pick) against 3, 4, 6 and 8 ways, 1.618
// ms per 512-token prefill against 1.666 / 1.625 / 1.620 / 1.624 ms.
template <int EPI, bool OUT8, int GM, int GN, int NW, int KT, int NS>
static void launch_mfma_kernel(LinearArgs& p, int mblocks, int nblocks, int splits, int kps, int32_t* part,
                               hipStream_t stream) {
  using T = MfmaTile<GM, GN, NW, KT, NS>;
  const int cus = current_cu_count();
  const int64_t tiles = (int64_t)mblocks * nblocks;
  // many rounds of workgroups (8 or more): persistent workgroups, as many as fit at once (one per
  // CU for the 256x256 tiles, whose ring fills the LDS), each stepping through its XCD's tiles.
  // Measured: 2048 x 896 x 151936 (18.6 rounds) 457 -> 447 us; 512 x 896 x 151936 (4.6 rounds)
  // 136 -> 147 us, so fewer rounds keep one workgroup per tile.
  const int per_cu = std::max(1, (160 * 1024) / T::LDS_BYTES);
  const bool persist = !part && tiles >= 8ll * cus * per_cu;
  const unsigned gx = persist ? (unsigned)(cus / 8 * 8 * per_cu) : (unsigned)(ceil_div(mblocks * nblocks, 8) * 8);
  hipLaunchKernelGGL((linear_mfma<EPI, OUT8, GM, GN, NW, KT, NS>), dim3(gx, splits), dim3(T::NT), T::LDS_BYTES, stream,
                     p, mblocks, nblocks, kps, part, persist ? 1 : 0);
}

// With norm (a resadd linear whose output rows are normalised and quantised next): a split-K
// launch finishes its planes with splitk_finish_norm_kernel and sets *norm_done.
template <int EPI, bool OUT8, int GM, int GN, int NW, int KT>
static int launch_mfma(LinearArgs& p, void* ws, hipStream_t stream, const NormQuant* norm = nullptr,
                       bool* norm_done = nullptr) {
  const int mblocks = (int)ceil_div(p.M, GM), nblocks = (int)ceil_div(p.N, GN);
  const int64_t tiles = (int64_t)mblocks * nblocks;
  const int k64 = (int)(p.K / 64), ktiles = (int)(p.K / KT);
  const int cus = current_cu_count();
  int splits = 1;
  // the finishing kernels store 4 (8) adjacent columns at once and read aux rows in 8-byte words
  const bool fin_ok = p.ldo % 4 == 0 && (uintptr_t)p.out % 8 == 0 && (!p.aux || (p.ldaux % 4 == 0 && (uintptr_t)p.aux % 8 == 0));
  if (ws && p.N % 4 == 0 && tiles < cus && fin_ok) {
    const int smax = (int)std::min<int64_t>(std::min<int64_t>(8, ceil_div(2 * cus, tiles)), k64 / 4);
    double best = 0.0;
    for (int sp = 2; sp <= smax; ++sp) {
      const double plane_bytes = (double)sp * p.M * p.N * 4;
      if (plane_bytes > (double)WS_SCRATCH_BYTES) break;
      const double gain = (GM * GN >= 128 * 128 ? 0.5 : 0.4) * k64 * (sp - 1) / sp - (5.0 + plane_bytes / 4e6);
      if (gain > best) {
        best = gain;
        splits = sp;
      }
    }
  }
  const int kps = (int)ceil_div(ktiles, splits);  // K tiles per split
  splits = (int)ceil_div(ktiles, kps);
  // an XCD's contiguous run of tiles shares one operand in its L2: the W panels (M-block fastest)
  // unless A is much taller than W (N-block fastest: an M-block's A rows are read once per XCD
  // instead of once per N-block).  Measured: 8192 x 896 x 896 14.0 -> 12.5 us, 8192 x 4864 x 896
  // 46.7 -> 41.4 us; at M / N = 2.3 (2048 rows) within +-2 %, so only from four times N
  p.nfast = p.M >= 4ll * p.N ? 1 : 0;
  p.nblk = nblocks;
  // M-fastest with more A than an XCD's 4 MiB L2 holds (a prompt batch's lm_head): groups of
  // M-blocks whose A rows take ~2 MiB, so an XCD's run of tiles keeps both its A group and its W
  // panels in L2
  p.mgroup = (int64_t)p.M * p.K > (4ll << 20) ? (int)std::max<int64_t>(1, (2ll << 20) / ((int64_t)GM * p.K)) : 0;
  int32_t* part = splits > 1 ? reinterpret_cast<int32_t*>(static_cast<char*>(ws) + WS_SCRATCH) : nullptr;
  if constexpr (deep_ring_fits<GM, GN, KT>()) {
    if (tiles * splits < cus)
      launch_mfma_kernel<EPI, OUT8, GM, GN, NW, KT, 3>(p, mblocks, nblocks, splits, kps, part, stream);
    else
      launch_mfma_kernel<EPI, OUT8, GM, GN, NW, KT, ring_stages<KT>()>(p, mblocks, nblocks, splits, kps, part, stream);
  } else {
    launch_mfma_kernel<EPI, OUT8, GM, GN, NW, KT, ring_stages<KT>()>(p, mblocks, nblocks, splits, kps, part, stream);
  }
  LLHIP_LAUNCH_CHECK();
  if (part) {
    if constexpr (EPI == EPI_RESADD && !OUT8) {
      if (norm && p.N % 8 == 0 && p.N <= NORM_MAX_K) {
        hipLaunchKernelGGL(splitk_finish_norm_kernel, dim3((unsigned)p.M), dim3(256), 0, stream, p, part, splits, *norm);
        LLHIP_LAUNCH_CHECK();
        *norm_done = true;
        return 0;
      }
    }
    const int64_t quads = (int64_t)p.M * p.N / 4;
    hipLaunchKernelGGL((linear_splitk_finish<EPI, OUT8>), dim3((unsigned)std::min<int64_t>(ceil_div(quads, 256), 8 * cus)),
                       dim3(256), 0, stream, p, part, splits);
    LLHIP_LAUNCH_CHECK();
  }
  return 0;
}

// The MFMA tile shape for a prompt-sized linear, over K tiles of KT bytes
template <int EPI, bool OUT8, int KT>
static int launch_mfma_shape(LinearArgs& p, void* ws, hipStream_t stream, const NormQuant* norm, bool* norm_done) {
  // 256x256 tiles when M fills them and they fill every CU.  The 256x256 kernel keeps 128
  // accumulators per lane at two waves per SIMD; the aux-reading epilogues would spill there.
  if constexpr (EPI == EPI_NONE) {
    if (p.M >= 256 && (int64_t)ceil_div(p.M, 256) * ceil_div(p.N, 256) >= current_cu_count())
      return launch_mfma<EPI, OUT8, 256, 256, 8, KT>(p, ws, stream);
  }
  // 128x128 tiles while they fill the CUs, else 64x128 tiles (twice as many workgroups, three per
  // CU), or 64x64 tiles (each workgroup streams half the W rows per K tile) while those take one
  // round of workgroups (512 x 896 x 896 7.9 -> 6.0 us, 512 x 4864 x 896 split along K 15.6 ->
  // 14.0 us), or two for a short K, where 64x128 tiles would run unsplit (2048 x 896 x 896 7.3 ->
  // 6.6 us; at K = 4864 two rounds of them lose to 64x128 split along K, 29.6 vs 25.9 us); split
  // along K when even those are too few
  const int cus = current_cu_count();
  if ((int64_t)ceil_div(p.M, 128) * ceil_div(p.N, 128) >= cus)
    return launch_mfma<EPI, OUT8, 128, 128, 4, KT>(p, ws, stream, norm, norm_done);
  const int64_t t64 = (int64_t)ceil_div(p.M, 64) * ceil_div(p.N, 64);
  if (t64 <= cus || (t64 <= 2ll * cus && p.K <= 1024))
    return launch_mfma<EPI, OUT8, 64, 64, 4, KT>(p, ws, stream, norm, norm_done);
  return launch_mfma<EPI, OUT8, 64, 128, 4, KT>(p, ws, stream, norm, norm_done);
}

template <int EPI, bool OUT8>
static int launch_linear(LinearArgs& p, void* ws, hipStream_t stream, const NormQuant* norm = nullptr,
                         bool* norm_done = nullptr) {
  const bool aligned = (p.K % 16 == 0) && (p.lda % 16 == 0) && ((uintptr_t)p.A % 16 == 0) && ((uintptr_t)p.W % 16 == 0);
  if (p.M >= 128 && p.K % 64 == 0 && aligned) {
    if (p.K % 128 == 0) return launch_mfma_shape<EPI, OUT8, 128>(p, ws, stream, norm, norm_done);
    return launch_mfma_shape<EPI, OUT8, 64>(p, ws, stream, norm, norm_done);
  }
  if (p.M > 16 && aligned) {
    // 128x256 block tiles when they still fill the chip, else 128x128
    const int mblocks = (int)ceil_div(p.M, 128);
    const int nb256 = (int)ceil_div(p.N, 256), nb128 = (int)ceil_div(p.N, 128);
    if ((int64_t)mblocks * nb256 >= 2 * current_cu_count())
      hipLaunchKernelGGL((linear_tiled<EPI, OUT8, 2, 4>), dim3(mblocks * nb256), dim3(256), 0, stream, p, mblocks, nb256);
    else
      hipLaunchKernelGGL((linear_tiled<EPI, OUT8, 2, 2>), dim3(mblocks * nb128), dim3(256), 0, stream, p, mblocks, nb128);
    LLHIP_LAUNCH_CHECK();
    return 0;
  }
  const int tiles = (int)ceil_div(p.N, 16);
  if (p.M == 1 && aligned && tiles < 2 * current_cu_count() && (int64_t)p.N * p.K < (1ll << 31)) {
    // lanes per column: enough chunks per lane to amortise the fold, at most G1_PF in flight
    const int nch = p.K / 16;
    if (nch >= 128) {
      hipLaunchKernelGGL((linear_gemv1<EPI, OUT8, 64>), dim3(p.N), dim3(64), 0, stream, p);
    } else if (nch >= 64) {
      hipLaunchKernelGGL((linear_gemv1<EPI, OUT8, 32>), dim3(ceil_div(p.N, 2)), dim3(64), 0, stream, p);
    } else if (nch >= 32) {
      hipLaunchKernelGGL((linear_gemv1<EPI, OUT8, 16>), dim3(ceil_div(p.N, 4)), dim3(64), 0, stream, p);
    } else if (nch >= 16) {
      hipLaunchKernelGGL((linear_gemv1<EPI, OUT8, 8>), dim3(ceil_div(p.N, 8)), dim3(64), 0, stream, p);
    } else {
      hipLaunchKernelGGL((linear_gemv1<EPI, OUT8, 4>), dim3(ceil_div(p.N, 16)), dim3(64), 0, stream, p);
    }
    LLHIP_LAUNCH_CHECK();
    return 0;
  }
  const int zblocks = (int)ceil_div(p.M, 16);
  const int cus = current_cu_count();
  int nw = 1;
  p.cpb = 16;
  if ((int64_t)tiles * zblocks >= cus) {
    // waves per workgroup: enough waves on the chip to keep HBM busy, never more than K steps
    while (nw < GEMV_MAX_WAVES && (int64_t)tiles * zblocks * nw * 2 <= 8 * cus && nw * 2 <= p.steps) nw *= 2;
  } else {
    // narrow output (a decode projection of a few rows): fewer columns per workgroup so that every
    // CU streams a share of W, and enough waves that each wave's K slice is loaded at entry
    while (p.cpb > 4 && ceil_div(p.N, p.cpb) * zblocks < cus) p.cpb /= 2;
    nw = (int)std::min<int64_t>(GEMV_MAX_WAVES, ceil_div(p.steps, GEMV_PF));
  }
  dim3 grid((unsigned)ceil_div(p.N, p.cpb), 1, zblocks);
  if (aligned)
    hipLaunchKernelGGL((linear_gemv<EPI, OUT8, true>), grid, dim3(64 * nw), 0, stream, p);
  else
    hipLaunchKernelGGL((linear_gemv<EPI, OUT8, false>), grid, dim3(64 * nw), 0, stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

// grouped launch of up to GROUP_MAX linears of one input (64x128 tiles); other shapes run the
// problems one by one through launch_linear
static int launch_linear_group(const LinearArgs& base, const llhip_linear_problem* pr, int count, void* ws,
                               hipStream_t s) {
  const bool aligned = (base.K % 64 == 0) && (base.lda % 16 == 0) && ((uintptr_t)base.A % 16 == 0);
  bool ok = aligned && count <= GROUP_MAX;
  for (int q = 0; ok && q < count; ++q) ok = (uintptr_t)pr[q].W % 16 == 0;
  if (!ok) {
    for (int q = 0; q < count; ++q) {
      LinearArgs p = base;
      p.W = static_cast<const int8_t*>(pr[q].W);
      p.rq = static_cast<const int32_t*>(pr[q].rq);
      p.bias = static_cast<const int32_t*>(pr[q].bias);
      p.out = pr[q].out;
      p.ldo = pr[q].ldo;
      p.N = (int)pr[q].N;
      const int rc = pr[q].out_i8 ? launch_linear<EPI_NONE, true>(p, ws, s) : launch_linear<EPI_NONE, false>(p, ws, s);
      if (rc) return rc;
    }
    return 0;
  }
  // 64x64 tiles while they take one round of workgroups (each workgroup streams half the W rows per
  // K tile), else 64x128
  const int mblocks = (int)ceil_div(base.M, 64), cus = current_cu_count();
  int64_t n64 = 0;
  for (int q = 0; q < count; ++q) n64 += ceil_div(pr[q].N, 64);
  const bool narrow = base.K % 128 == 0 && mblocks * n64 <= cus;
  const int gn = narrow ? 64 : 128;
  LinearGroup g{};
  g.count = count;
  g.nb0[0] = 0;
  for (int q = 0; q < count; ++q) {
    g.W[q] = static_cast<const int8_t*>(pr[q].W);
    g.rq[q] = static_cast<const int32_t*>(pr[q].rq);
    g.bias[q] = static_cast<const int32_t*>(pr[q].bias);
    g.out[q] = pr[q].out;
    g.ldo[q] = pr[q].ldo;
    g.N[q] = (int)pr[q].N;
    g.out8[q] = pr[q].out_i8 ? 1 : 0;
    g.nb0[q + 1] = g.nb0[q] + (int)ceil_div(pr[q].N, gn);
  }
  const dim3 grid((unsigned)(ceil_div((int64_t)mblocks * g.nb0[count], 8) * 8));
  if (narrow) {
    using T = MfmaTile<64, 64, 4, 128, 3>;
    hipLaunchKernelGGL((linear_mfma_group<64, 64, 4, 128, 3>), grid, dim3(T::NT), T::LDS_BYTES, s, base, g, mblocks);
  } else if (base.K % 128 == 0 && grid.x < (unsigned)cus) {
    using T = MfmaTile<64, 128, 4, 128, 3>;
    hipLaunchKernelGGL((linear_mfma_group<64, 128, 4, 128, 3>), grid, dim3(T::NT), T::LDS_BYTES, s, base, g, mblocks);
  } else if (base.K % 128 == 0) {
    using T = MfmaTile<64, 128, 4, 128>;
    hipLaunchKernelGGL((linear_mfma_group<64, 128, 4, 128, T::NS>), grid, dim3(T::NT), T::LDS_BYTES, s, base, g, mblocks);
  } else {
    using T = MfmaTile<64, 128, 4, 64>;
    hipLaunchKernelGGL((linear_mfma_group<64, 128, 4, 64, T::NS>), grid, dim3(T::NT), T::LDS_BYTES, s, base, g, mblocks);
  }
  LLHIP_LAUNCH_CHECK();
  return 0;
}

// exact int64 A . int8 W^T (golden.py:217-240 computes the same integers through FP64 BLAS)
__global__ void exact_matmul_kernel(const int64_t* A, int64_t M, int64_t K, const int8_t* W, int64_t N, int64_t* out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx % N;
  int64_t acc = 0;
  for (int64_t k = 0; k < K; ++k) acc += wmul(A[m * K + k], (int64_t)W[n * K + k]);
  out[idx] = acc;
}

}  // namespace llhip

using namespace llhip;

// llhip_linear's checks and kernel arguments (rc 1: nothing to compute)
static int linear_args(LinearArgs& p, const int8_t* A, int64_t M, int64_t K, int64_t lda, const int8_t* W, int64_t N,
                       const int32_t* rq, const int32_t* bias, int epilogue, const int16_t* aux, int64_t ldaux,
                       int64_t aux_shift, int64_t silu_Mi, int64_t silu_Si, int64_t silu_sh, int out_i8, void* out,
                       int64_t ldo) {
  if (M < 0 || N < 0 || K < 0) return fail(-EINVAL, "linear: negative shape");
  if (M == 0 || N == 0) return 1;
  if (K > 65535) return fail(-EINVAL, "linear: K=%lld exceeds the int32 accumulator bound 65535", (long long)K);
  if (M > INT32_MAX || N > INT32_MAX) return fail(-EINVAL, "linear: shape too large");
  if (lda < K || ldo < N) return fail(-EINVAL, "linear: leading dimension too small");
  if (!A || !W || !rq || !out) return fail(-EINVAL, "linear: null operand");
  if (epilogue < 0 || epilogue > 3) return fail(-EINVAL, "linear: unknown epilogue %d", epilogue);
  if (out_i8 && epilogue != EPI_NONE) return fail(-EINVAL, "i8 output is only valid with epilogue none");
  if ((epilogue == EPI_RESADD || epilogue == EPI_MUL) && (!aux || ldaux < N))
    return fail(-EINVAL, "linear: epilogue needs aux [M][N]");
  if (epilogue == EPI_MUL && !shift_ok(aux_shift)) return fail(-EINVAL, "linear: aux_shift out of [0,63]");
  if (epilogue == EPI_SILU && (!shift_ok(silu_Si) || !shift_ok(silu_sh)))
    return fail(-EINVAL, "linear: silu shift out of [0,63]");
  if (epilogue == EPI_SILU && !u32_ok(silu_Mi)) return fail(-EINVAL, "linear: silu Mi must be u32");
  p.A = A;
  p.W = W;
  p.rq = rq;
  p.bias = bias;
  p.aux = aux;
  p.out = out;
  p.lda = lda;
  p.ldaux = ldaux;
  p.ldo = ldo;
  p.Mi = silu_Mi;
  p.M = (int)M;
  p.K = (int)K;
  p.N = (int)N;
  p.aux_shift = (int)aux_shift;
  p.Si = (int)silu_Si;
  p.sh = (int)silu_sh;
  p.steps = (int)ceil_div(K, 64);
  if (p.steps == 0) p.steps = 1;
  return 0;
}

extern "C" int llhip_linear(const int8_t* A, int64_t M, int64_t K, int64_t lda, const int8_t* W, int64_t N,
                            const int32_t* rq, const int32_t* bias, int epilogue, const int16_t* aux, int64_t ldaux,
                            int64_t aux_shift, int64_t silu_Mi, int64_t silu_Si, int64_t silu_sh, int out_i8,
                            void* out, int64_t ldo, void* ws, void* stream) {
  LinearArgs p{};
  const int rc = linear_args(p, A, M, K, lda, W, N, rq, bias, epilogue, aux, ldaux, aux_shift, silu_Mi, silu_Si, silu_sh,
                             out_i8, out, ldo);
  if (rc) return rc < 0 ? rc : 0;
  hipStream_t s = (hipStream_t)stream;
  if (out_i8) return launch_linear<EPI_NONE, true>(p, ws, s);
  switch (epilogue) {
    case EPI_RESADD: return launch_linear<EPI_RESADD, false>(p, ws, s);
    case EPI_SILU: return launch_linear<EPI_SILU, false>(p, ws, s);
    case EPI_MUL: return launch_linear<EPI_MUL, false>(p, ws, s);
    default: return launch_linear<EPI_NONE, false>(p, ws, s);
  }
}

extern "C" int llhip_linear_norm(const int8_t* A, int64_t M, int64_t K, int64_t lda, const int8_t* W, int64_t N,
                                 const int32_t* rq, const int32_t* bias, const int16_t* aux, int64_t ldaux, int16_t* out,
                                 int64_t ldo, const llhip_norm_quant_desc* norm, void* ws, void* stream) {
  if (!norm) return fail(-EINVAL, "linear_norm: null descriptor");
  NormQuant pr{};
  int rc = fill_pre(pr, *norm);
  if (rc) return rc;
  if (norm->prequant || norm->x != out || norm->ldx != ldo || norm->K != N || (!norm->h_out && !norm->hq_out))
    return fail(-EINVAL, "linear_norm: the norm must read the linear's output rows [M][N] and write a result");
  LinearArgs p{};
  rc = linear_args(p, A, M, K, lda, W, N, rq, bias, EPI_RESADD, aux, ldaux, 0, 0, 0, 0, 0, out, ldo);
  if (rc) return rc < 0 ? rc : 0;
  bool done = false;
  rc = launch_linear<EPI_RESADD, false>(p, ws, (hipStream_t)stream, &pr, &done);
  if (rc || done) return rc;
  return llhip_rmsnorm_quant(norm, M, stream);
}

extern "C" int llhip_gate_up(const llhip_gate_up_desc* d, void* stream) {
  if (!d) return fail(-EINVAL, "gate_up: null descriptor");
  const int64_t M = d->M, K = d->K, N = d->N;
  if (M < 0 || K < 0 || N < 0 || M > INT32_MAX || N > INT32_MAX || d->lda < K || d->ld < N)
    return fail(-EINVAL, "gate_up: bad shape");
  if (K > 65535) return fail(-EINVAL, "linear: K=%lld exceeds the int32 accumulator bound 65535", (long long)K);
  if (!d->A || !d->Wg || !d->Wu || !d->rqg || !d->rqu || !d->fq_out) return fail(-EINVAL, "gate_up: null operand");
  if (!u32_ok(d->silu_Mi) || !shift_ok(d->silu_Si) || !shift_ok(d->silu_sh) || !shift_ok(d->mul_sh) ||
      !u32_ok(d->fq_M) || !shift_ok(d->fq_S))
    return fail(-EINVAL, "gate_up: parameter out of range");
  if (M == 0 || N == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  LinearArgs p{};
  p.A = static_cast<const int8_t*>(d->A);
  p.lda = d->lda;
  p.M = (int)M;
  p.K = (int)K;
  p.N = (int)N;
  p.steps = (int)std::max<int64_t>(ceil_div(K, 64), 1);
  p.Mi = d->silu_Mi;
  p.Si = (int)d->silu_Si;
  p.sh = (int)d->silu_sh;
  const bool fits = K % 64 == 0 && K > 0 && d->lda % 16 == 0 && (uintptr_t)d->A % 16 == 0 && (uintptr_t)d->Wg % 16 == 0 &&
                    (uintptr_t)d->Wu % 16 == 0;
  if (!fits) {  // the three ops one by one
    if (!d->sg_out || !d->f_out)
      return fail(-EINVAL, "gate_up: sg_out and f_out may be NULL only when K %% 64 == 0 and A, lda, Wg, Wu are "
                           "16-byte aligned");
    p.W = static_cast<const int8_t*>(d->Wg);
    p.rq = static_cast<const int32_t*>(d->rqg);
    p.bias = static_cast<const int32_t*>(d->bg);
    p.out = d->sg_out;
    p.ldo = d->ld;
    int rc = launch_linear<EPI_SILU, false>(p, nullptr, s);
    if (rc) return rc;
    p.W = static_cast<const int8_t*>(d->Wu);
    p.rq = static_cast<const int32_t*>(d->rqu);
    p.bias = static_cast<const int32_t*>(d->bu);
    p.aux = static_cast<const int16_t*>(d->sg_out);
    p.ldaux = d->ld;
    p.aux_shift = (int)d->mul_sh;
    p.out = d->f_out;
    if ((rc = launch_linear<EPI_MUL, false>(p, nullptr, s))) return rc;
    for (int64_t m = 0; m < M; ++m)
      if ((rc = llhip_quant(static_cast<const int16_t*>(d->f_out) + m * d->ld, N, d->fq_M, d->fq_S,
                            static_cast<int8_t*>(d->fq_out) + m * d->ld, stream)))
        return rc;
    return 0;
  }
  p.W = static_cast<const int8_t*>(d->Wg);
  p.rq = static_cast<const int32_t*>(d->rqg);
  p.bias = static_cast<const int32_t*>(d->bg);
  DualArgs a{};
  a.Wu = static_cast<const int8_t*>(d->Wu);
  a.rqu = static_cast<const int32_t*>(d->rqu);
  a.bu = static_cast<const int32_t*>(d->bu);
  a.sg = static_cast<int16_t*>(d->sg_out);
  a.f = static_cast<int16_t*>(d->f_out);
  a.fq = static_cast<int8_t*>(d->fq_out);
  a.ld = d->ld;
  a.fqM = d->fq_M;
  a.fqS = (int)d->fq_S;
  a.mul_sh = (int)d->mul_sh;
  const int mblocks = (int)ceil_div(M, 64);
  // tiles M-block fastest (consecutive workgroups share the gate and up panels), the M-blocks in
  // groups of ~2 MiB of A rows when A exceeds an XCD's 4 MiB L2 (a prompt batch)
  p.mgroup = M * K > (4ll << 20) ? (int)std::max<int64_t>(1, (2ll << 20) / (64 * K)) : 0;
  // 64x64 tiles (48 KB rings) while they number at most three per CU (512 x 896 x 4864
  // 18.6 -> 17.6 us, 256 rows 14.1 -> 12.6 us), else 64x128
  if (p.K % 128 == 0 && (int64_t)mblocks * ceil_div(N, 64) <= 3ll * current_cu_count()) {
    const int nblocks = (int)ceil_div(N, 64);
    p.nblk = nblocks;
    const dim3 grid((unsigned)(ceil_div((int64_t)mblocks * nblocks, 8) * 8));
    hipLaunchKernelGGL((linear_mfma_dual<128, 2, 64>), grid, dim3(512), 2 * (64 + 2 * 64) * 128, s, p, a, mblocks,
                       nblocks);
    LLHIP_LAUNCH_CHECK();
    return 0;
  }
  const int nblocks = (int)ceil_div(N, 128);
  p.nblk = nblocks;
  const dim3 grid((unsigned)(ceil_div((int64_t)mblocks * nblocks, 8) * 8));
  if (p.K % 128 == 0)
    hipLaunchKernelGGL((linear_mfma_dual<128, 2>), grid, dim3(512), 2 * (64 + 2 * 128) * 128, s, p, a, mblocks, nblocks);
  else
    hipLaunchKernelGGL((linear_mfma_dual<64, GSTAGES>), grid, dim3(512), GSTAGES * (64 + 2 * 128) * 64, s, p, a, mblocks,
                       nblocks);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

// one rope descriptor of llhip_linear_group_rope: the checks of llhip_rope_quant for rows produced by
// problem pr (x = pr.out, D = 64, the problem's N = H D), plus the alignments of the 16- and 8-byte
// accesses of the epilogue
static int rope_group_part(const llhip_rope_quant_desc& d, const llhip_linear_problem& pr, int64_t M, bool key) {
  if (d.D != 64 || d.H < 1 || d.H * 64 != pr.N || d.x != pr.out || d.M != M || d.ldx != pr.ldo || pr.out_i8)
    return fail(-EINVAL, "linear_group_rope: the rope rows must be problem %s's i16 output, head_dim 64", key ? "k" : "q");
  if (!u32_ok(d.qM) || !shift_ok(d.qS)) return fail(-EINVAL, "linear_group_rope: quant multiplier must be u32, shift in [0,63]");
  if (!d.yq || !d.cos_tab || !d.sin_tab) return fail(-EINVAL, "linear_group_rope: null operand");
  if (d.seq_rows < 0 || (d.seq_rows > 0 && (d.pos_dev || d.row_pos || M % d.seq_rows)))
    return fail(-EINVAL, "linear_group_rope: sequences of seq_rows rows need M %% seq_rows == 0 and no row positions");
  const int64_t span = d.seq_rows > 0 ? d.seq_rows : M;
  if (!d.pos_dev && !d.row_pos && (d.pos < 0 || d.pos + span > d.table_rows))
    return fail(-ERANGE, "rope: positions exceed the table");
  const auto al = [](const void* p, uintptr_t a) { return (uintptr_t)p % a == 0; };
  if (!al(pr.out, 16) || pr.ldo % 8 || !al(d.y, 16) || !al(d.yq, 8) || !al(d.cos_tab, 16) || !al(d.sin_tab, 16))
    return fail(-EINVAL, "linear_group_rope: misaligned rows or tables");
  if (!key) {
    if (d.kc || d.vc) return fail(-EINVAL, "linear_group_rope: the query rows write no cache");
    return 0;
  }
  if (!d.kc != !d.vc) return fail(-EINVAL, "linear_group_rope: the key rows write both caches or neither");
  if (d.kc) {
    if (!d.pos_dev && !d.row_pos && d.pos + span > d.max_seq)
      return fail(-ERANGE, "positions %lld..%lld exceed max_seq=%lld", (long long)d.pos, (long long)(d.pos + span - 1),
                  (long long)d.max_seq);
    if ((d.row_pos || d.seq_rows > 0) && d.slot_stride < d.H * d.max_seq * 64)
      return fail(-EINVAL, "linear_group_rope: cache slots overlap");
    if (!al(d.kc, 16) || !al(d.vc, 16) || d.slot_stride % 16) return fail(-EINVAL, "linear_group_rope: misaligned caches");
  }
  return 0;
}

extern "C" int llhip_linear_group_rope(const int8_t* A, int64_t M, int64_t K, int64_t lda, const llhip_linear_problem* probs,
                                       const llhip_rope_quant_desc* rq, const llhip_rope_quant_desc* rk, void* ws,
                                       void* stream) {
  (void)ws;
  if (!probs || !rq || !rk || !A) return fail(-EINVAL, "linear_group_rope: null argument");
  if (M < 1 || M > INT32_MAX || K < 128 || K % 128 || K > 65535 || lda < K || lda % 16 || (uintptr_t)A % 16)
    return fail(-EINVAL, "linear_group_rope: rows of K %% 128 == 0 bytes, 16-byte aligned");
  for (int q = 0; q < 3; ++q) {
    const llhip_linear_problem& r = probs[q];
    if (r.N < 64 || r.N % 64 || r.N > INT32_MAX || r.ldo < r.N || !r.W || !r.rq || !r.out || (uintptr_t)r.W % 16)
      return fail(-EINVAL, "linear_group_rope: bad problem %d (N a multiple of 64, 16-byte aligned weights)", q);
  }
  const llhip_linear_problem& pv = probs[2];
  if (!pv.out_i8 || pv.N != probs[1].N || (uintptr_t)pv.out % 16 || pv.ldo % 16)
    return fail(-EINVAL, "linear_group_rope: the v problem writes i8 rows of the k problem's width, 16-byte aligned");
  int rc = rope_group_part(*rq, probs[0], M, false);
  if (!rc) rc = rope_group_part(*rk, probs[1], M, true);
  if (rc) return rc;
  if (rk->kc && (rk->v != pv.out || rk->ldv != pv.ldo))
    return fail(-EINVAL, "linear_group_rope: the V cache rows must be problem v's output");
  if (rq->pos != rk->pos || rq->pos_dev != rk->pos_dev || rq->row_pos != rk->row_pos || rq->seq_rows != rk->seq_rows ||
      rq->cos_tab != rk->cos_tab || rq->sin_tab != rk->sin_tab || rq->table_rows != rk->table_rows)
    return fail(-EINVAL, "linear_group_rope: q and k rows at different positions");
  LinearArgs p{};
  p.A = A;
  p.lda = lda;
  p.M = (int)M;
  p.K = (int)K;
  p.steps = (int)ceil_div(K, 64);
  const int mblocks = (int)ceil_div(M, 64), cus = current_cu_count();
  const int64_t n64 = (probs[0].N + probs[1].N + probs[2].N) / 64;
  const bool narrow = mblocks * n64 <= cus;
  const int gn = narrow ? 64 : 128;
  LinearGroup g{};
  g.count = 3;
  g.nb0[0] = 0;
  for (int q = 0; q < 3; ++q) {
    g.W[q] = static_cast<const int8_t*>(probs[q].W);
    g.rq[q] = static_cast<const int32_t*>(probs[q].rq);
    g.bias[q] = static_cast<const int32_t*>(probs[q].bias);
    g.out[q] = probs[q].out;
    g.ldo[q] = probs[q].ldo;
    g.N[q] = (int)probs[q].N;
    g.out8[q] = probs[q].out_i8 ? 1 : 0;
    g.nb0[q + 1] = g.nb0[q] + (int)ceil_div(probs[q].N, gn);
  }
  const llhip_rope_quant_desc* rd[2] = {rq, rk};
  for (int q = 0; q < 2; ++q) {
    g.rope[q].kind = 1;
    g.rope[q].qM = rd[q]->qM;
    g.rope[q].qS = (int)rd[q]->qS;
    g.rope[q].y = static_cast<int16_t*>(rd[q]->y);
    g.rope[q].yq = static_cast<int8_t*>(rd[q]->yq);
    g.rope[q].cache = static_cast<int8_t*>(rd[q]->kc);
  }
  g.rope[2].kind = 2;
  g.rope[2].cache = static_cast<int8_t*>(rk->vc);
  g.rs.cos_tab = static_cast<const int16_t*>(rk->cos_tab);
  g.rs.sin_tab = static_cast<const int16_t*>(rk->sin_tab);
  g.rs.pos_dev = static_cast<const int32_t*>(rk->pos_dev);
  g.rs.row_pos = static_cast<const int32_t*>(rk->row_pos);
  g.rs.table_rows = rk->table_rows;
  g.rs.max_seq = rk->max_seq;
  g.rs.slot_stride = rk->slot_stride;
  g.rs.seq_rows = rk->seq_rows;
  g.rs.pos = (int)rk->pos;
  const dim3 grid((unsigned)(ceil_div((int64_t)mblocks * g.nb0[3], 8) * 8));
  const hipStream_t s = (hipStream_t)stream;
  if (narrow) {
    using T = MfmaTile<64, 64, 4, 128, 3>;
    hipLaunchKernelGGL((linear_mfma_group<64, 64, 4, 128, 3, true>), grid, dim3(T::NT), T::LDS_BYTES, s, p, g, mblocks);
  } else if (grid.x < (unsigned)cus) {
    using T = MfmaTile<64, 128, 4, 128, 3>;
    hipLaunchKernelGGL((linear_mfma_group<64, 128, 4, 128, 3, true>), grid, dim3(T::NT), T::LDS_BYTES, s, p, g, mblocks);
  } else {
    using T = MfmaTile<64, 128, 4, 128>;
    hipLaunchKernelGGL((linear_mfma_group<64, 128, 4, 128, T::NS, true>), grid, dim3(T::NT), T::LDS_BYTES, s, p, g,
                       mblocks);
  }
  LLHIP_LAUNCH_CHECK();
  return 0;
}

extern "C" int llhip_linear_group(const int8_t* A, int64_t M, int64_t K, int64_t lda, int64_t count,
                                  const llhip_linear_problem* probs, void* ws, void* stream) {
  if (M < 0 || K < 0 || count < 0) return fail(-EINVAL, "linear_group: negative shape");
  if (count > GROUP_MAX) return fail(-EINVAL, "linear_group: at most %d problems", GROUP_MAX);
  if (count && !probs) return fail(-EINVAL, "linear_group: null problems");
  if (K > 65535) return fail(-EINVAL, "linear: K=%lld exceeds the int32 accumulator bound 65535", (long long)K);
  if (M > INT32_MAX || lda < K || !A) return fail(-EINVAL, "linear_group: bad input rows");
  for (int64_t q = 0; q < count; ++q) {
    const llhip_linear_problem& r = probs[q];
    if (r.N < 0 || r.N > INT32_MAX || r.ldo < r.N || !r.W || !r.rq || !r.out)
      return fail(-EINVAL, "linear_group: bad problem %lld", (long long)q);
  }
  if (M == 0 || count == 0) return 0;
  LinearArgs p{};
  p.A = A;
  p.lda = lda;
  p.M = (int)M;
  p.K = (int)K;
  p.steps = (int)std::max<int64_t>(ceil_div(K, 64), 1);
  // problems with N = 0 take no tiles
  llhip_linear_problem live[GROUP_MAX];
  int n = 0;
  for (int64_t q = 0; q < count; ++q)
    if (probs[q].N > 0) live[n++] = probs[q];
  if (n == 0) return 0;
  return launch_linear_group(p, live, n, ws, (hipStream_t)stream);
}

extern "C" int llhip_exact_matmul(const int64_t* A, int64_t M, int64_t K, const int8_t* W, int64_t N, int64_t* out,
                                  void* stream) {
  if (M < 0 || N < 0 || K < 0) return fail(-EINVAL, "exact_matmul: negative shape");
  if (M == 0 || N == 0) return 0;
  const int64_t total = M * N;
  hipLaunchKernelGGL(exact_matmul_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, A, M,
                     K, W, N, out);
  LLHIP_LAUNCH_CHECK();
  return 0;
}
