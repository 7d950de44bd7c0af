// attn engine of libllhip: KV-cache write (golden.py:344-351) and causal GQA
// integer attention (golden.py:353-366 over attention_head golden.py:162-180,
// NUMERICS.md "Attention").
//
// The integer softmax needs three reductions over all T keys in order -- the
// maximum score, the sum of LUT exponentials (which depend on that maximum) and
// the probability-weighted value sum (which depends on the sum through inv) --
// so it cannot be computed online per tile.  Each of them is an exact integer
// reduction, so any reduction order gives the reference's result.
//
// attention_rowhead: one 512-thread block per (row m, query head h).  Scores for
// all T keys are staged in LDS (int32), block reductions give max and sum, and
// the value pass splits the head dimension into 16-byte chunks across threads
// and the keys across thread groups (four keys in flight per thread); partial
// sums are folded across lanes with shuffles, then across waves in LDS.
#include <algorithm>
#include <mutex>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {


constexpr int ATTN_MAX_T = 12000;  // 48 KB of scores + 32 KB of value partials (D = 256) in LDS

struct AttnArgs {
  const int8_t* q;
  const int8_t* kc;
  const int8_t* vc;
  int8_t* out;
  const int32_t* pos_dev;
  const int32_t* row_pos;  // per-row positions (row m in cache slot m), or null
  int64_t slot_stride;
  int seq_rows;  // > 0: rows of seq_rows each per sequence (row m at pos + m % seq_rows, slot m / seq_rows)
  int64_t ldq, ldo, max_seq;
  int64_t Ms, Mo;
  int Ss, So;
  int H, Hkv, pos, pb;
  int lds_T;  // score slots in LDS
  int M;
  // decode chain (WO kernels, one row): the output projection's partial sums of each head,
  // wo_acc[n] += sum_d out[h D + d] * Wo[n][h D + d] with the panel wop[h][n][d] = Wo[n][h D + d],
  // and the accumulator rows of the next projection cleared by head 0
  const int8_t* wop;
  int32_t* wo_acc;
  int32_t* zero;
  int wo_N, zero_n;
  int span;  // dimension-slice launches of one row: XCDs per GQA group (0: one, the grid below)
};

// clear n int32 values from one workgroup (16-byte aligned)
__device__ __forceinline__ void zero_words(int32_t* p, int n) {
  if (!p) return;
  for (int i = 4 * (int)threadIdx.x; i < n; i += 4 * (int)blockDim.x) {
    if (i + 4 <= n) *reinterpret_cast<v4i*>(p + i) = v4i{0, 0, 0, 0};
    else
      for (int j = i; j < n; ++j) p[j] = 0;
  }
}

// sum over aligned groups of DC consecutive lanes (DC in 1..16), every lane ending with its
// group's total (DPP butterfly within a 16-lane row)
template <int DC>
__device__ __forceinline__ int32_t chunk_sum(int32_t v) {
  if constexpr (DC >= 2) v += dpp_mov<DPP_QUAD_XOR1>(v);
  if constexpr (DC >= 4) v += dpp_mov<DPP_QUAD_XOR2>(v);
  if constexpr (DC >= 8) v += dpp_mov<DPP_HALF_MIRROR>(v);
  if constexpr (DC >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
  return v;
}

__device__ __forceinline__ int32_t dot16(const v4i& a, const v4i& b) {
  int32_t s = __builtin_amdgcn_sdot4(a.x, b.x, 0, false);
  s = __builtin_amdgcn_sdot4(a.y, b.y, s, false);
  s = __builtin_amdgcn_sdot4(a.z, b.z, s, false);
  return __builtin_amdgcn_sdot4(a.w, b.w, s, false);
}

// The output projection's partial sums of head h from its D output bytes in LDS (one row).  Lane l
// takes 16-byte chunk l % DC of panel column n (64 / DC consecutive columns per wave load, so the
// loads are contiguous); the DC lanes of a column add their products and the first one adds the
// column's sum into the accumulators.  wpre holds this thread's first NPF chunks.
// Columns [n_lo, n_hi) of the output projection's partial sums of head h from its D output bytes
// in LDS (one row).  Lane l takes 16-byte chunk l % DC of a panel column (64 / DC consecutive
// columns per wave load, so the loads are contiguous); the DC lanes of a column add their products
// and the first one adds the column's sum into the accumulators.  wpre holds this thread's first
// NPF chunks (wo_prefetch).
template <int D, int NPF>
__device__ __forceinline__ void wo_partial(const AttnArgs& p, int h, const int8_t* ah, const v4i* wpre, int n_lo,
                                           int n_hi) {
  constexpr int DC = D / 16;
  const int lane = threadIdx.x & 63, kc = lane % DC;
  const int cpb = (int)(blockDim.x / DC);  // columns per block-wide load
  const int c0 = n_lo + (int)(threadIdx.x / DC);
  const v4i a = *reinterpret_cast<const v4i*>(ah + 16 * kc);
#pragma unroll
  for (int i = 0; i < NPF; ++i) {
    const int n = c0 + i * cpb;
    const int32_t s = chunk_sum<DC>(dot16(a, wpre[i]));
    if (kc == 0 && n < n_hi && s != 0) atomic_add_dev(p.wo_acc + n, s);
  }
  // the rest four loads at a time (all in flight before the first is used)
  const Rsrc wr = rsrc(p.wop + (int64_t)h * p.wo_N * D, (int64_t)p.wo_N * D);
  for (int n0 = NPF * cpb; c0 - (int)(threadIdx.x / DC) + n0 < n_hi; n0 += 4 * cpb) {
    v4i w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = c0 + n0 + u * cpb;
      w[u] = ld16(wr, n < n_hi ? (uint32_t)(n * D + 16 * kc) : LD_OOB);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = c0 + n0 + u * cpb;
      const int32_t s = chunk_sum<DC>(dot16(a, w[u]));
      if (kc == 0 && n < n_hi && s != 0) atomic_add_dev(p.wo_acc + n, s);
    }
  }
}

// this thread's first NPF chunks of head h's output-projection panel for columns from n_lo
template <int D, int NPF>
__device__ __forceinline__ void wo_prefetch(const AttnArgs& p, int h, v4i* wpre, int n_lo, int n_hi) {
  constexpr int DC = D / 16;
  const int kc = (threadIdx.x & 63) % DC, cpb = (int)(blockDim.x / DC), c0 = n_lo + (int)(threadIdx.x / DC);
  const Rsrc wr = rsrc(p.wop + (int64_t)h * p.wo_N * D, (int64_t)p.wo_N * D);
#pragma unroll
  for (int i = 0; i < NPF; ++i) {
    const int n = c0 + i * cpb;
    wpre[i] = ld16(wr, n < n_hi ? (uint32_t)(n * D + 16 * kc) : LD_OOB);
  }
}

constexpr int ATTN_THREADS = 512;
constexpr int ATTN_WAVES = ATTN_THREADS / 64;
constexpr int SLICE_WPF = 2;  // output-projection columns per thread loaded at entry by a slice workgroup

// Output-projection partial sums of the 16 head dimensions [16 ds, 16 ds + 16) of head h (their
// requantised outputs in ah): each thread takes whole panel columns n = tid, tid + 512, ... (one
// 16-byte chunk each; the first SLICE_WPF of them loaded at entry into wpre).
template <int D>
__device__ __forceinline__ void wo_slice(const AttnArgs& p, int h, int ds, const int8_t* ah, const v4i* wpre) {
  const v4i a = *reinterpret_cast<const v4i*>(ah);
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < SLICE_WPF; ++i) {
    const int n = tid + i * ATTN_THREADS;
    const int32_t s = dot16(a, wpre[i]);
    if (n < p.wo_N && s != 0) atomic_add_dev(p.wo_acc + n, s);
  }
  const Rsrc wr = rsrc(p.wop + (int64_t)h * p.wo_N * D, (int64_t)p.wo_N * D);
  for (int n0 = SLICE_WPF * ATTN_THREADS + tid; n0 < p.wo_N; n0 += 4 * ATTN_THREADS) {
    v4i w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = n0 + u * ATTN_THREADS;
      w[u] = ld16(wr, n < p.wo_N ? (uint32_t)(n * D + 16 * ds) : LD_OOB);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = n0 + u * ATTN_THREADS;
      const int32_t s = dot16(a, w[u]);
      if (n < p.wo_N && s != 0) atomic_add_dev(p.wo_acc + n, s);
    }
  }
}

__device__ __forceinline__ int32_t sbyte(int w, int i) { return (int32_t)(int8_t)((uint32_t)w >> (8 * i)); }

template <int D>
__device__ __forceinline__ int32_t dot_row(const v4i* qv, const v4i* kv) {
  constexpr int DC = D / 16;
  int32_t s = 0;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    s = __builtin_amdgcn_sdot4(qv[c].x, kv[c].x, s, false);
    s = __builtin_amdgcn_sdot4(qv[c].y, kv[c].y, s, false);
    s = __builtin_amdgcn_sdot4(qv[c].z, kv[c].z, s, false);
    s = __builtin_amdgcn_sdot4(qv[c].w, kv[c].w, s, false);
  }
  return s;
}

// sum over the lanes of a 16-lane row that share lane % DC (DC divides 16)
template <int DC>
__device__ __forceinline__ int32_t row_fold(int32_t v) {
  if constexpr (DC <= 1) v += dpp_mov<DPP_ROW_ROR + 1>(v);
  if constexpr (DC <= 2) v += dpp_mov<DPP_ROW_ROR + 2>(v);
  if constexpr (DC <= 4) v += dpp_mov<DPP_ROW_ROR + 4>(v);
  if constexpr (DC <= 8) v += dpp_mov<DPP_ROW_ROR + 8>(v);
  return v;
}

// exp LUTs staged in LDS: kExpI (16 u16 = 8 dwords) then kExpF (256 u16 = 128 dwords)
constexpr int LUT_DW = 136;

__device__ __forceinline__ uint32_t lut_prob_lds(int64_t z, const uint16_t* ei, const uint16_t* ef) {
  if (z >= 4096 || z < 0) return 0u;
  const uint32_t zi = (uint32_t)z;
  return ((uint32_t)ei[zi >> 8] * (uint32_t)ef[zi & 255] + 32768u) >> 16;
}

// Loads at entry, in order of use: q and the keys of the first score pass, the LUT dwords (wave
// 0), then the value rows of this thread's first VPF keys, so each phase waits only for its own
// group and the value latency hides behind the score and softmax phases.  Keys >= T read zeros.
// SLICE (output-projection fold, one row): D / 16 workgroups per head, workgroup ds computing the
// head's full softmax but only the 16 output dimensions [16 ds, 16 ds + 16) and their share of the
// output projection -- each workgroup streams all keys but a sixteenth-byte slice of every value row
// and of the panel, so a head's value and panel bytes are spread over D / 16 CUs.
template <int D, bool WO, bool SLICE = false>
__global__ __launch_bounds__(ATTN_THREADS) void attention_rowhead(AttnArgs p) {
  static_assert(!SLICE || WO, "dimension slices fold the output projection");
  kernarg_warm<sizeof(AttnArgs)>();
  extern __shared__ int32_t sc[];  // [lds_T] scores, then probabilities
  __shared__ int32_t redmax[ATTN_WAVES], redsum[ATTN_WAVES];
  __shared__ uint32_t lut32[LUT_DW];
  __shared__ int32_t wpart[4 * ATTN_WAVES][D];
  __shared__ __attribute__((aligned(16))) int8_t ah[WO ? D : 16];
  // output-projection panel chunks per thread loaded ahead (covering 1024 columns x D bytes)
  constexpr int WPF = SLICE ? SLICE_WPF : WO ? (D <= 128 ? (1024 * (D / 16)) / ATTN_THREADS : 16) : 0;
  constexpr int DC = D / 16;  // 16-byte chunks per key row
  constexpr int DS = SLICE ? DC : 1;        // workgroups per head
  constexpr int VDC = SLICE ? 1 : DC;       // value chunks per key across the threads
  constexpr int TG = ATTN_THREADS / VDC;    // keys per block-wide value load
  constexpr int VPF = SLICE ? 2 : 8;

  // The G = H/Hkv query heads that read one (row, GQA group)'s K/V run on one XCD and share its
  // L2 (workgroup b is dispatched to XCD b % 8): pair u = m * Hkv + g goes to XCD u % 8, as
  // workgroups b = u % 8 + 8 * ((u / 8) * G + j) for its heads j.  The grid is
  // 8 * ceil(M * Hkv / 8) * G; workgroups past the last pair exit.
  // (With slices the grid has DS workgroups per head: j = (xk % (G * DS)) / DS, ds = xk % DS.)
  // A slice launch with span P > 1 (one row, Hkv * P = 8) spreads group g over the P XCDs
  // g * P .. g * P + P - 1 instead: its G * DS workgroups w sit at b = g * P + w % P + 8 * (w / P),
  // so all eight XCDs (their L2 and their CUs) serve the row and the grid has no idle workgroups.
  const int G = p.H / p.Hkv;
  int m, g, h, ds;
  if (SLICE && p.span > 1) {
    const int x = (int)(blockIdx.x % 8), w = x % p.span + p.span * (int)(blockIdx.x / 8);
    g = x / p.span;
    if (g >= p.Hkv || w >= G * DS) return;
    m = 0;
    h = g * G + w / DS;
    ds = w % DS;
  } else {
    const int xk = (int)(blockIdx.x / 8);
    const int u = (int)(blockIdx.x % 8) + 8 * (xk / (G * DS));
    if (u >= p.M * p.Hkv) return;
    m = u / p.Hkv;
    g = u % p.Hkv;
    h = g * G + (xk % (G * DS)) / DS;
    ds = xk % DS;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  // Loads in order of use: q and the keys of the first score pass, the LUT dwords (wave 0), the
  // value rows of this thread's first VPF keys.  The cache rows are addressed over the whole cache,
  // so these loads do not wait for the device position; rows at or past T are masked out below
  // (their scores are never kept, their probabilities are zero).
  const int64_t slot = p.row_pos ? m * p.slot_stride : 0;
  const int8_t* kbase = p.kc + slot + (int64_t)g * p.max_seq * D;
  const int8_t* vbase = p.vc + slot + (int64_t)g * p.max_seq * D;
  const Rsrc qr = rsrc(p.q + (int64_t)m * p.ldq + (int64_t)h * D, D);
  const Rsrc kr = rsrc(kbase, (int64_t)p.max_seq * D), vr = rsrc(vbase, (int64_t)p.max_seq * D);
  // Score pass layout: lane l takes 16-byte chunk kc = l % DC of key kw + i * KPB, so one wave load
  // covers 64 / DC consecutive keys (1 KiB contiguous) and the DC lanes of a key add their partial
  // dot products with DPP.  The first KPF loads per lane are issued here.
  constexpr int KPB = (64 / DC) * ATTN_WAVES;              // keys per block-wide load
  constexpr int KPF = (D <= 128 ? 1024 : 512) / KPB;      // loads per lane issued at entry
  const int kc = lane % DC, kw = wave * (64 / DC) + lane / DC;
  const v4i qc = ld16(qr, 16 * kc);
  v4i kpf[KPF];
#pragma unroll
  for (int i = 0; i < KPF; ++i) kpf[i] = ld16(kr, (uint32_t)((i * KPB + kw) * D + 16 * kc));
  issue_fence();
  uint32_t lw[3] = {0u, 0u, 0u};
  if (wave == 0) {  // (a load instruction costs address-unit cycles even when it reads nothing)
    const Rsrc ir = rsrc(kExpI, sizeof(kExpI)), fr = rsrc(kExpF, sizeof(kExpF));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int idx = lane + 64 * i;
      const bool mine = idx < LUT_DW;
      // one of the two reads is out of range (zero)
      lw[i] = (uint32_t)ld4(ir, mine && idx < 8 ? 4 * idx : LD_OOB) |
              (uint32_t)ld4(fr, mine && idx >= 8 ? 4 * (idx - 8) : LD_OOB);
    }
  }
  issue_fence();
  const int dc = SLICE ? ds : tid % DC, tg = tid / VDC;
  v4i vpre[VPF];
#pragma unroll
  for (int u = 0; u < VPF; ++u) vpre[u] = ld16(vr, (uint32_t)((tg + u * TG) * D + 16 * dc));
  issue_fence();
  // row m's context T = position + 1 (row m of a launch at pos sits at pos + m; with per-row
  // positions, row m is its own sequence in cache slot m), never past the cache.  A scalar load
  // issued after the vector loads: a wait for it waits for every earlier scalar load.
  const int T = min((p.row_pos ? *(const __attribute__((address_space(4))) int32_t*)(p.row_pos + m)
                               : load_pos(p.pos_dev, p.pos) + m) + 1,
                    (int)p.max_seq);
  if (WO && h == 0 && m == 0 && ds == 0) zero_words(p.zero, p.zero_n);

  // scores s[t] = q . k[t] (int32, |s| <= D * 2^14)
  int32_t lmax = INT32_MIN;
#pragma unroll
  for (int i = 0; i < KPF; ++i) {
    const int t = i * KPB + kw;
    const int32_t sv = chunk_sum<DC>(dot16(qc, kpf[i]));
    if (kc == 0 && t < T) {
      sc[t] = sv;
      lmax = max(lmax, sv);
    }
  }
  for (int t0 = KPF * KPB; t0 < T; t0 += 4 * KPB) {
    v4i kv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) kv[u] = ld16(kr, (uint32_t)((t0 + u * KPB + kw) * D + 16 * kc));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u * KPB + kw;
      const int32_t sv = chunk_sum<DC>(dot16(qc, kv[u]));
      if (kc == 0 && t < T) {
        sc[t] = sv;
        lmax = max(lmax, sv);
      }
    }
  }
  // the output-projection panel columns of this thread, requested once the score loads are
  // consumed: they are needed last and their loads overlap the softmax and the value pass
  v4i wpre[WPF > 0 ? WPF : 1];
  if constexpr (SLICE) {
    const Rsrc wr = rsrc(p.wop + (int64_t)h * p.wo_N * D, (int64_t)p.wo_N * D);
#pragma unroll
    for (int i = 0; i < WPF; ++i) {
      const int n = tid + i * ATTN_THREADS;
      wpre[i] = ld16(wr, n < p.wo_N ? (uint32_t)(n * D + 16 * ds) : LD_OOB);
    }
  } else if constexpr (WPF > 0) {
    wo_prefetch<D, WPF>(p, h, wpre, 0, p.wo_N);
  }
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
      if (lane + 64 * i < LUT_DW) lut32[lane + 64 * i] = lw[i];
  }
  lmax = wave_max_i32(lmax);
  if (lane == 0) redmax[wave] = lmax;
  __syncthreads();
  int32_t mx = redmax[0];
#pragma unroll
  for (int w = 1; w < ATTN_WAVES; ++w) mx = max(mx, redmax[w]);

  // p[t] = LUT(mulshift(mx - s[t], Ms, Ss)), then the sum
  const uint16_t* ei = reinterpret_cast<const uint16_t*>(lut32);
  const uint16_t* ef = ei + 16;
  uint32_t lsum = 0;
  for (int t = tid; t < T; t += ATTN_THREADS) {
    const uint32_t pr = lut_prob_lds(mulshift((int64_t)mx - sc[t], p.Ms, p.Ss), ei, ef);
    sc[t] = (int32_t)pr;
    lsum += pr;
  }
  lsum = (uint32_t)wave_sum_i32((int)lsum);  // T * 65535 < 2^31
  if (lane == 0) redsum[wave] = (int32_t)lsum;
  __syncthreads();
  uint32_t total = 0;
#pragma unroll
  for (int w = 0; w < ATTN_WAVES; ++w) total += (uint32_t)redsum[w];
  const uint32_t inv = 0x80000000u / (total > 1u ? total : 1u);  // 2^31 / total (golden.py:174)
  const int32_t cap = (1 << p.pb) - 1;
  const int shp = 31 - p.pb;
  for (int t = tid; t < T; t += ATTN_THREADS) {
    const int64_t pn = rshr((int64_t)sc[t] * (int64_t)inv, shp);
    sc[t] = (int32_t)(pn < cap ? pn : cap);
  }
  __syncthreads();

  // o[d] = sum_t pn[t] * v[t][d]: thread (tg, dc) takes keys tg, tg+TG, ... (prefetched rows
  // first, then four in flight)
  int32_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0;
#pragma unroll
  for (int u = 0; u < VPF; ++u) {
    const int t = tg + u * TG;
    const int32_t pn = t < T ? sc[t] : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] += pn * sbyte(vpre[u].x, i);
      acc[4 + i] += pn * sbyte(vpre[u].y, i);
      acc[8 + i] += pn * sbyte(vpre[u].z, i);
      acc[12 + i] += pn * sbyte(vpre[u].w, i);
    }
  }
  for (int ta = tg + VPF * TG; ta < T; ta += 4 * TG) {
    v4i vv[4];
    int32_t pn[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = ta + u * TG;
      vv[u] = ld16(vr, (uint32_t)(t * D + 16 * dc));
      pn[u] = t < T ? sc[t] : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] += pn[u] * sbyte(vv[u].x, i);
        acc[4 + i] += pn[u] * sbyte(vv[u].y, i);
        acc[8 + i] += pn[u] * sbyte(vv[u].z, i);
        acc[12 + i] += pn[u] * sbyte(vv[u].w, i);
      }
  }
  // the lanes of a 16-lane row with equal lane % VDC hold the same 16 columns: fold them with
  // row rotations, then the 4 rows x ATTN_WAVES partials in LDS
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = row_fold<VDC>(acc[i]);
  if ((lane & 15) < VDC) {
#pragma unroll
    for (int i = 0; i < 16; ++i) wpart[wave * 4 + (lane >> 4)][16 * (lane & 15) + i] = acc[i];
  }
  __syncthreads();
  for (int d = tid; d < (SLICE ? 16 : D); d += ATTN_THREADS) {
    int32_t o = 0;
#pragma unroll
    for (int w = 0; w < 4 * ATTN_WAVES; ++w) o += wpart[w][d];
    if (p.pb == 15) o = rshr32(o, 7);
    const int8_t y = (int8_t)sat8(mulshift(o, p.Mo, p.So));
    p.out[(int64_t)m * p.ldo + (int64_t)h * D + 16 * ds + d] = y;
    if constexpr (WO) ah[d] = y;
  }
  if constexpr (SLICE) {
    __syncthreads();
    wo_slice<D>(p, h, ds, ah, wpre);
  } else if constexpr (WO) {
    __syncthreads();
    wo_partial<D, WPF>(p, h, ah, wpre, 0, p.wo_N);
  }
}

// ---------------------------------------------------------------------------------------
// attention_tiled: M >= 2 rows at consecutive positions pos.. (prefill, chunked prefill)
// ---------------------------------------------------------------------------------------
// One workgroup per (block of 16 query rows, query head); its waves split the 64-key tiles of the
// block's context.  Each of the three reductions is one pass over the tiles, and every pass
// recomputes the tile's scores with v_mfma_i32_16x16x64_i8 (cheap next to a round trip of the
// scores through LDS):
//   S^T = K . Q^T : A = 16 key rows, B = the 16 query rows, so lane (lg = lane / 16, lr = lane % 16)
//                   holds query row lr's scores of keys 16j + 4lg + r (subtile j, register r);
//   O = P . V     : A = P with row lr and byte 4j + r <-> key 16j + 4lg + r -- exactly the score
//                   layout, so the probabilities never leave the lane -- and B = V^T in the same key
//                   order, made by multiplying 16-key blocks of V (as A) by 0/1 selection matrices:
//                   C[key][n] = V[key][16e + n], which lands key 16b + 4lg + r, column 16e + lr in
//                   lane (lg, lr) register r.
// The probabilities pn < 2^15 enter the int8 MFMA as base-128 digits (pn = d0 + 128 d1 + 16384 d2,
// each digit in [0, 127]), so O = O0 + 128 O1 + 16384 O2 is the exact integer sum.  The operand
// byte order inside a lane (which K index a byte feeds) is the same for A and B, so neither
// product depends on it.  Keys at or past a row's T get probability 0; keys past the block's last
// row read zeros.
constexpr int AT_ROWS = 16;
constexpr int AT_MIN_M = 2;       // launches of fewer rows use attention_rowhead
constexpr int AT_MAX_T = 32767;   // per-row sum of T probabilities < 2^31
constexpr int AT_SPLIT_MIN_TILES = 32;  // contexts of >= 2048 keys may be split across workgroups
constexpr int AT_SPLIT_MAXS = 128;      // splits per (row block, head) pair

template <int D>
struct AttnTileCfg {
  static constexpr int DK = (D + 63) / 64;  // 64-byte K chunks of a key row
  static constexpr int DB = D / 16;         // 16-column blocks of the output
  static constexpr int MAXW = D <= 128 ? 8 : 4;
  static constexpr int SC = D <= 64 ? 2 : 1;  // tiles per wave whose scores stay in registers
};

__device__ __forceinline__ uint32_t pack4(int32_t a, int32_t b, int32_t c, int32_t d) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
  return lo | hi;
}

// Probability of a key x = mx - s >= 0 below the row maximum (golden.py:170-172):
// z = rshr(x * Ms, Ss) = (x * Ms + 2^(Ss-1)) >> Ss for x >= 0 (x < 2^24, Ms < 2^32: one 32x32->64
// multiply-add), p = 0 past the 4096-entry exponent range, else the rounded LUT product.
struct ProbParams {
  uint32_t Ms;
  int Ss;
  uint64_t zc;  // 2^(Ss-1), or 0 when Ss = 0
};

__device__ __forceinline__ uint32_t prob_lds(int32_t x, const ProbParams& q, const uint16_t* ei, const uint16_t* ef) {
  const uint64_t z = ((uint64_t)(uint32_t)x * q.Ms + q.zc) >> q.Ss;
  if (z >= 4096) return 0u;
  const uint32_t zi = (uint32_t)z;
  return ((uint32_t)ei[zi >> 8] * (uint32_t)ef[zi & 255] + 32768u) >> 16;
}

// MINW: waves per SIMD the register budget must allow.  4 (at most 128 VGPRs) for launches of more
// waves than fit three to a SIMD: one batched prefill of 16 x 512 rows, 76.9 vs 82.7 us per layer;
// a single prompt's few workgroups all fit anyway and run faster without the cap (10.16 vs 10.56 us).
template <int D, int MINW = 1>
__global__ __launch_bounds__(64 * AttnTileCfg<D>::MAXW, MINW) void attention_tiled(AttnArgs p) {
  using C = AttnTileCfg<D>;
  constexpr int DK = C::DK, DB = C::DB, SC = C::SC;
  __shared__ uint32_t lut32[LUT_DW];
  __shared__ int32_t red[C::MAXW][AT_ROWS];
  __shared__ int32_t osum[AT_ROWS][D];
  // With Hkv a multiple of 8, GQA group g runs on XCD g % 8 (workgroup b is dispatched to XCD
  // b % 8) so its query heads share that XCD's L2; otherwise heads are numbered in order (an
  // XCD-per-group mapping would leave most workgroups empty).
  const int G = p.H / p.Hkv;
  int h;
  if (p.Hkv % 8 == 0) {
    const int g = (int)(blockIdx.x % 8) + 8 * (int)((blockIdx.x / 8) / G);
    h = g * G + (int)((blockIdx.x / 8) % G);
  } else {
    h = (int)blockIdx.x;
  }
  const int g = h / G;
  const int m0 = blockIdx.y * AT_ROWS;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int nw = blockDim.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  int pos = load_pos(p.pos_dev, p.pos);
  int64_t slot = 0;
  if (p.seq_rows > 0) {  // a block of sequence b = m0 / seq_rows (seq_rows % 16 == 0): its own caches
    const int b = m0 / p.seq_rows;
    pos -= b * p.seq_rows;
    slot = (int64_t)b * p.slot_stride;
  }
  const int mlast = min(m0 + AT_ROWS, p.M) - 1;
  const int Tb = min(pos + mlast + 1, (int)p.max_seq);  // keys any row of the block sees
  const int ntiles = (Tb + 63) >> 6;
  const int m = m0 + lr;  // this lane's query row
  const int tlim = m < p.M ? min(pos + m + 1, (int)p.max_seq) : 0;
  const int8_t* kbase = p.kc + slot + (int64_t)g * p.max_seq * D;
  const int8_t* vbase = p.vc + slot + (int64_t)g * p.max_seq * D;
  const Rsrc kr = rsrc(kbase, (int64_t)Tb * D), vr = rsrc(vbase, (int64_t)Tb * D);

  v4i qf[DK];
  {
    const Rsrc qr = rsrc(p.q + (int64_t)m0 * p.ldq + (int64_t)h * D, (int64_t)AT_ROWS * p.ldq);
#pragma unroll
    for (int c = 0; c < DK; ++c)
      qf[c] = ld16(qr, (m < p.M && 64 * c + 16 * lg < D) ? (uint32_t)(lr * p.ldq + 64 * c + 16 * lg) : LD_OOB);
  }
  // the LUT words (words tid, tid + blockDim.x, ..., at least 64 threads; stored to LDS once the tile
  // loads below are issued, so the two round trips overlap)
  constexpr int LUTW = (LUT_DW + 63) / 64;
  uint32_t lutw[LUTW];
  {
    const Rsrc ir = rsrc(kExpI, sizeof(kExpI)), fr = rsrc(kExpF, sizeof(kExpF));
#pragma unroll
    for (int i = 0; i < LUTW; ++i) {
      const int idx = tid + i * (int)blockDim.x;
      lutw[i] = (uint32_t)ld4(ir, idx < 8 ? 4 * idx : LD_OOB) | (uint32_t)ld4(fr, idx >= 8 && idx < LUT_DW ? 4 * (idx - 8) : LD_OOB);
    }
  }
  // K (or V) fragment of 16-key block j of tile kt: key kt*64 + 16j + lr, bytes [64c + 16lg, +16)
  auto frag_off = [&](int kt, int j, int c) -> uint32_t {
    return 64 * c + 16 * lg < D ? (uint32_t)((kt * 64 + 16 * j + lr) * D + 64 * c + 16 * lg) : LD_OOB;
  };
  auto kfrags = [&](int kt, v4i (&kf)[4][DK]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < DK; ++c) kf[j][c] = ld16(kr, frag_off(kt, j, c));
  };
  auto score_mfmas = [&](const v4i (&kf)[4][DK], v4i (&st)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      st[j] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < DK; ++c) st[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[j][c], qf[c], st[j], 0, 0, 0);
    }
  };
  auto scores = [&](int kt, v4i (&st)[4]) {
    v4i kf[4][DK];
    kfrags(kt, kf);
    score_mfmas(kf, st);
  };
  // key of subtile j, register r of tile kt in this lane
  auto key = [&](int kt, int j, int r) { return kt * 64 + 16 * j + 4 * lg + r; };

  // Tiles wave + it * nw (it < SC) keep their scores, later their probabilities, in registers
  // across the three passes; further tiles are recomputed in each pass.
  v4i cache[SC][4];
  // values of the cached tiles, requested with their keys (used in pass 3)
  v4i vcache[SC][4][DK];

  // pass 1: row maxima.  The cached tiles' keys and values are requested first, then the LUT and
  // the output sums are staged in LDS (visible after the first barrier).
  int32_t vmax = INT32_MIN;
  v4i kfc[SC][4][DK];
#pragma unroll
  for (int it = 0; it < SC; ++it) {
    const int kt = wave + it * nw;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < DK; ++c) kfc[it][j][c] = ld16(kr, kt < ntiles ? frag_off(kt, j, c) : LD_OOB);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < DK; ++c) vcache[it][j][c] = ld16(vr, kt < ntiles ? frag_off(kt, j, c) : LD_OOB);
  }
#pragma unroll
  for (int i = 0; i < LUTW; ++i) {
    const int idx = tid + i * (int)blockDim.x;
    if (idx < LUT_DW) lut32[idx] = lutw[i];
  }
  for (int idx = tid; idx < AT_ROWS * D; idx += blockDim.x) (&osum[0][0])[idx] = 0;
#pragma unroll
  for (int it = 0; it < SC; ++it) {
    const int kt = wave + it * nw;
    if (kt < ntiles) {
      score_mfmas(kfc[it], cache[it]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (key(kt, j, r) < tlim) vmax = max(vmax, cache[it][j][r]);
    }
  }
  for (int kt = wave + SC * nw; kt < ntiles; kt += nw) {
    v4i st[4];
    scores(kt, st);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (key(kt, j, r) < tlim) vmax = max(vmax, st[j][r]);
  }
  vmax = max(vmax, __shfl_xor(vmax, 16));
  vmax = max(vmax, __shfl_xor(vmax, 32));
  if (lg == 0) red[wave][lr] = vmax;
  __syncthreads();
  int32_t mx = red[0][lr];
  for (int w = 1; w < nw; ++w) mx = max(mx, red[w][lr]);
  __syncthreads();

  // pass 2: sums of the LUT exponentials (cached tiles keep p in place of s)
  const uint16_t* ei = reinterpret_cast<const uint16_t*>(lut32);
  const uint16_t* ef = ei + 16;
  ProbParams pq;
  pq.Ms = (uint32_t)p.Ms;
  pq.Ss = p.Ss;
  pq.zc = p.Ss > 0 ? 1ull << (p.Ss - 1) : 0ull;
  // a tile's 16 scores -> probabilities in place (0 at or past the row's T), returning their sum:
  // branch-free, all 32 LUT reads issued before the first is used
  auto tile_probs = [&](int kt, v4i (&st)[4]) -> uint32_t {
    uint32_t zi[16], lo[16], hi[16];
    bool ok[16];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint64_t z = ((uint64_t)(uint32_t)(mx - st[j][r]) * pq.Ms + pq.zc) >> pq.Ss;
        ok[4 * j + r] = key(kt, j, r) < tlim && z < 4096;
        zi[4 * j + r] = ok[4 * j + r] ? (uint32_t)z : 0u;
      }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      hi[k] = ei[zi[k] >> 8];
      lo[k] = ef[zi[k] & 255];
    }
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = 4 * j + r;
        const uint32_t pr = ok[k] ? (hi[k] * lo[k] + 32768u) >> 16 : 0u;
        st[j][r] = (int32_t)pr;
        sum += pr;
      }
    return sum;
  };
  uint32_t vsum = 0;
#pragma unroll
  for (int it = 0; it < SC; ++it) {
    const int kt = wave + it * nw;
    if (kt < ntiles) vsum += tile_probs(kt, cache[it]);
  }
  for (int kt = wave + SC * nw; kt < ntiles; kt += nw) {
    v4i st[4];
    scores(kt, st);
    vsum += tile_probs(kt, st);
  }
  vsum += (uint32_t)__shfl_xor((int)vsum, 16);
  vsum += (uint32_t)__shfl_xor((int)vsum, 32);
  if (lg == 0) red[wave][lr] = (int32_t)vsum;
  __syncthreads();
  uint32_t total = 0;
  for (int w = 0; w < nw; ++w) total += (uint32_t)red[w][lr];
  const uint32_t inv = 0x80000000u / (total > 1u ? total : 1u);  // 2^31 / total (golden.py:174)
  const uint32_t cap = (1u << p.pb) - 1u;
  const int shp = 31 - p.pb;
  const uint64_t pc = 1ull << (shp - 1);  // rounding constant of rshr(p * inv, 31 - pb), shp >= 16
  const bool three = p.pb > 14;           // pn >= 2^14 possible: a third digit

  // 0/1 selection matrix e: lane (lg, lr) has byte lr set when lg == e
  v4i sel[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t bit = lg == e ? 1u << (8 * (lr & 3)) : 0u;
    sel[e] = v4i{(lr >> 2) == 0 ? (int)bit : 0, (lr >> 2) == 1 ? (int)bit : 0, (lr >> 2) == 2 ? (int)bit : 0,
                 (lr >> 2) == 3 ? (int)bit : 0};
  }

  // pass 3: O = P . V
  v4i oacc[DB];
#pragma unroll
  for (int e = 0; e < DB; ++e) oacc[e] = v4i{0, 0, 0, 0};
  // probabilities (already zero for keys a row does not see) -> base-128 digits -> MFMAs
  auto pv_tile = [&](const v4i (&pr)[4], const v4i (&vf)[4][DK]) {
    v4i pd[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t pn[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t v = (uint32_t)(((uint64_t)(uint32_t)pr[j][r] * inv + pc) >> shp);
        pn[r] = v < cap ? v : cap;
      }
      pd[0][j] = (int)pack4(pn[0] & 127, pn[1] & 127, pn[2] & 127, pn[3] & 127);
      pd[1][j] = (int)pack4((pn[0] >> 7) & 127, (pn[1] >> 7) & 127, (pn[2] >> 7) & 127, (pn[3] >> 7) & 127);
      pd[2][j] = (int)pack4(pn[0] >> 14, pn[1] >> 14, pn[2] >> 14, pn[3] >> 14);
    }
#pragma unroll
    for (int e = 0; e < DB; ++e) {
      const int c = e >> 2;
      v4i vt;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const v4i t = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf[b][c], sel[e & 3], v4i{0, 0, 0, 0}, 0, 0, 0);
        vt[b] = (int)pack4(t[0], t[1], t[2], t[3]);
      }
      const v4i a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(pd[0], vt, v4i{0, 0, 0, 0}, 0, 0, 0);
      const v4i a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(pd[1], vt, v4i{0, 0, 0, 0}, 0, 0, 0);
      const v4i a2 = three ? __builtin_amdgcn_mfma_i32_16x16x64_i8(pd[2], vt, v4i{0, 0, 0, 0}, 0, 0, 0) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; ++r) oacc[e][r] += a0[r] + 128 * a1[r] + 16384 * a2[r];
    }
  };
#pragma unroll
  for (int it = 0; it < SC; ++it)
    if (wave + it * nw < ntiles) pv_tile(cache[it], vcache[it]);
  for (int kt = wave + SC * nw; kt < ntiles; kt += nw) {
    v4i vf[4][DK];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int c = 0; c < DK; ++c) vf[b][c] = ld16(vr, frag_off(kt, b, c));
    v4i st[4];
    scores(kt, st);
    tile_probs(kt, st);
    pv_tile(st, vf);
  }
  // C layout of O: lane (lg, lr) register r = row 4lg + r, column 16e + lr
#pragma unroll
  for (int e = 0; e < DB; ++e)
#pragma unroll
    for (int r = 0; r < 4; ++r) atomicAdd(&osum[4 * lg + r][16 * e + lr], oacc[e][r]);
  __syncthreads();
  for (int idx = tid; idx < AT_ROWS * D; idx += blockDim.x) {
    const int row = idx / D, d = idx % D;
    if (m0 + row >= p.M) break;
    int32_t o = osum[row][d];
    if (p.pb == 15) o = rshr32(o, 7);
    p.out[(int64_t)(m0 + row) * p.ldo + (int64_t)h * D + d] = (int8_t)sat8(mulshift(o, p.Mo, p.So));
  }
}

// ---------------------------------------------------------------------------------------
// attention_split: long contexts with few (row block, head) pairs.  The 64-key tiles of the
// context are split over S workgroups per pair and the three reductions become three launches
// (PHASE 1: row maxima, 2: sums of the LUT exponentials, 3: probability-weighted value sums),
// each writing per-split partials to the workspace, then attention_split_finish adds the value
// partials and requantises.  Every partial is an exact integer max or sum, so the split changes
// no result.  The per-tile arithmetic is that of attention_tiled (16 query rows per workgroup,
// S^T = K . Q^T, V^T by selection MFMAs, base-128 probability digits).
// ONE (a single query row, the decode launch): phase 1 also stores the row's scores (4 bytes per
// key), and phase 3 sums the LUT exponentials of all of them itself -- every workgroup of a head
// reads the head's T scores -- so phase 2 and its launch are not needed.
// ---------------------------------------------------------------------------------------
struct SplitWs {
  int32_t* maxv;  // [pairs][S][16]
  int32_t* sumv;  // [pairs][S][16]
  int32_t* outv;  // [pairs][S][16][D]
  int32_t* sc;    // ONE: [pairs][ntiles * 64] scores of row 0
};

template <int D>
__device__ __forceinline__ SplitWs split_ws(int32_t* ws, int64_t pairs, int S) {
  SplitWs w;
  w.maxv = ws;
  w.sumv = ws + pairs * S * AT_ROWS;
  w.outv = ws + 2 * pairs * S * AT_ROWS;
  w.sc = w.outv + pairs * S * AT_ROWS * D;
  return w;
}

template <int D, int PHASE, bool ONE>
__global__ __launch_bounds__(64 * AttnTileCfg<D>::MAXW) void attention_split(AttnArgs p, int S, int tps, int32_t* ws) {
  using C = AttnTileCfg<D>;
  constexpr int DK = C::DK, DB = C::DB;
  __shared__ uint32_t lut32[LUT_DW];
  __shared__ int32_t red[C::MAXW][AT_ROWS];
  __shared__ int32_t osum[PHASE == 3 ? AT_ROWS : 1][PHASE == 3 ? D : 1];
  __shared__ int32_t spart[PHASE >= 2 ? AT_SPLIT_MAXS : 1][AT_ROWS];  // every split's maxima (then sums)
  const int G = p.H / p.Hkv;
  int h;
  if (p.Hkv % 8 == 0) {
    const int g = (int)(blockIdx.x % 8) + 8 * (int)((blockIdx.x / 8) / G);
    h = g * G + (int)((blockIdx.x / 8) % G);
  } else {
    h = (int)blockIdx.x;
  }
  const int g = h / G;
  const int rb = blockIdx.y, z = blockIdx.z;
  const int64_t pairs = (int64_t)p.H * gridDim.y;
  const int64_t pair = (int64_t)h * gridDim.y + rb;
  const SplitWs w = split_ws<D>(ws, pairs, S);
  const int m0 = rb * AT_ROWS;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int nw = blockDim.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int pos = load_pos(p.pos_dev, p.pos);
  const int mlast = min(m0 + AT_ROWS, p.M) - 1;
  const int Tb = min(pos + mlast + 1, (int)p.max_seq);
  const int ntiles = (Tb + 63) >> 6;
  const int kt0 = z * tps, kt1 = min(kt0 + tps, ntiles);  // this split's tiles (possibly none)
  const int m = m0 + lr;
  const int tlim = m < p.M ? min(pos + m + 1, (int)p.max_seq) : 0;
  const int8_t* kbase = p.kc + (int64_t)g * p.max_seq * D;
  const int8_t* vbase = p.vc + (int64_t)g * p.max_seq * D;
  const Rsrc kr = rsrc(kbase, (int64_t)Tb * D), vr = rsrc(vbase, (int64_t)Tb * D);

  v4i qf[DK];
  {
    const Rsrc qr = rsrc(p.q + (int64_t)m0 * p.ldq + (int64_t)h * D, (int64_t)AT_ROWS * p.ldq);
#pragma unroll
    for (int c = 0; c < DK; ++c)
      qf[c] = ld16(qr, (m < p.M && 64 * c + 16 * lg < D) ? (uint32_t)(lr * p.ldq + 64 * c + 16 * lg) : LD_OOB);
  }
  // ONE, phase 3: row 0's scores of the first SPF * blockDim keys, loaded before anything waits
  constexpr int SPF = (ONE && PHASE == 3) ? 16 : 1;
  const int t0 = min(pos + 1, (int)p.max_seq);
  const Rsrc scr = rsrc(w.sc + pair * ((int64_t)ntiles * 64), (int64_t)t0 * 4);
  int32_t sv[SPF];
  if constexpr (ONE && PHASE == 3) {
#pragma unroll
    for (int u = 0; u < SPF; ++u) {
      const int k = tid + u * (int)blockDim.x;
      sv[u] = ld4(scr, k < t0 ? (uint32_t)(4 * k) : LD_OOB);
    }
  }
  if (PHASE >= 2) {
    const Rsrc ir = rsrc(kExpI, sizeof(kExpI)), fr = rsrc(kExpF, sizeof(kExpF));
    for (int idx = tid; idx < LUT_DW; idx += blockDim.x)
      lut32[idx] = (uint32_t)ld4(ir, idx < 8 ? 4 * idx : LD_OOB) | (uint32_t)ld4(fr, idx >= 8 ? 4 * (idx - 8) : LD_OOB);
  }
  if (PHASE == 3)
    for (int idx = tid; idx < AT_ROWS * D; idx += blockDim.x) (&osum[0][0])[idx] = 0;
  auto frag_off = [&](int kt, int j, int c) -> uint32_t {
    return 64 * c + 16 * lg < D ? (uint32_t)((kt * 64 + 16 * j + lr) * D + 64 * c + 16 * lg) : LD_OOB;
  };
  auto scores = [&](int kt, v4i (&st)[4]) {
    v4i kf[4][DK];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < DK; ++c) kf[j][c] = ld16(kr, frag_off(kt, j, c));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      st[j] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < DK; ++c) st[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[j][c], qf[c], st[j], 0, 0, 0);
    }
  };
  auto key = [&](int kt, int j, int r) { return kt * 64 + 16 * j + 4 * lg + r; };

  if (PHASE == 1) {
    int32_t vmax = INT32_MIN;
    int32_t* scrow = w.sc + pair * ((int64_t)ntiles * 64);
    for (int kt = kt0 + wave; kt < kt1; kt += nw) {
      v4i st[4];
      scores(kt, st);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (key(kt, j, r) < tlim) {
            vmax = max(vmax, st[j][r]);
            if (ONE && lr == 0) scrow[key(kt, j, r)] = st[j][r];
          }
    }
    vmax = max(vmax, __shfl_xor(vmax, 16));
    vmax = max(vmax, __shfl_xor(vmax, 32));
    if (lg == 0) red[wave][lr] = vmax;
    __syncthreads();
    if (tid < AT_ROWS) {
      int32_t mx = red[0][tid];
      for (int q = 1; q < nw; ++q) mx = max(mx, red[q][tid]);
      w.maxv[(pair * S + z) * AT_ROWS + tid] = mx;
    }
    return;
  }

  // row maximum over all splits (the S x 16 partials staged in LDS by the whole workgroup)
  for (int idx = tid; idx < S * AT_ROWS; idx += blockDim.x) (&spart[0][0])[idx] = w.maxv[pair * S * AT_ROWS + idx];
  __syncthreads();  // partials and LUT staged
  int32_t mx = INT32_MIN;
  for (int q = 0; q < S; ++q) mx = max(mx, spart[q][lr]);
  const uint16_t* ei = reinterpret_cast<const uint16_t*>(lut32);
  const uint16_t* ef = ei + 16;
  ProbParams pq;
  pq.Ms = (uint32_t)p.Ms;
  pq.Ss = p.Ss;
  pq.zc = p.Ss > 0 ? 1ull << (p.Ss - 1) : 0ull;

  if (PHASE == 2) {
    uint32_t vsum = 0;
    for (int kt = kt0 + wave; kt < kt1; kt += nw) {
      v4i st[4];
      scores(kt, st);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (key(kt, j, r) < tlim) vsum += prob_lds(mx - st[j][r], pq, ei, ef);
    }
    vsum += (uint32_t)__shfl_xor((int)vsum, 16);
    vsum += (uint32_t)__shfl_xor((int)vsum, 32);
    if (lg == 0) red[wave][lr] = (int32_t)vsum;
    __syncthreads();
    if (tid < AT_ROWS) {
      uint32_t t = 0;
      for (int q = 0; q < nw; ++q) t += (uint32_t)red[q][tid];
      w.sumv[(pair * S + z) * AT_ROWS + tid] = (int32_t)t;
    }
    return;
  }

  // PHASE 3: the row's total over all splits -> inv, then this split's P . V
  uint32_t total = 0;
  if constexpr (ONE) {
    // row 0's total from its stored scores, every thread a share of the keys (the first SPF of
    // them already in registers)
    int32_t mx0 = INT32_MIN;
    for (int q = 0; q < S; ++q) mx0 = max(mx0, spart[q][0]);
    uint32_t vs = 0;
    const int bd = (int)blockDim.x;
#pragma unroll
    for (int u = 0; u < SPF; ++u)
      if (tid + u * bd < t0) vs += prob_lds(mx0 - sv[u], pq, ei, ef);
    for (int k0 = tid + SPF * bd; k0 < t0; k0 += 8 * bd) {
      int32_t sb[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) sb[u] = ld4(scr, k0 + u * bd < t0 ? (uint32_t)(4 * (k0 + u * bd)) : LD_OOB);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u * bd < t0) vs += prob_lds(mx0 - sb[u], pq, ei, ef);
    }
    for (int o = 32; o > 0; o >>= 1) vs += (uint32_t)__shfl_xor((int)vs, o);
    __syncthreads();  // every lane has read spart (the maxima)
    if (lane == 0) red[wave][0] = (int32_t)vs;
    __syncthreads();
    for (int q = 0; q < nw; ++q) total += (uint32_t)red[q][0];
    if (lr != 0) total = 0;  // rows past M have no keys
  } else {
    __syncthreads();  // every lane has its maximum
    for (int idx = tid; idx < S * AT_ROWS; idx += blockDim.x) (&spart[0][0])[idx] = w.sumv[pair * S * AT_ROWS + idx];
    __syncthreads();
    for (int q = 0; q < S; ++q) total += (uint32_t)spart[q][lr];
  }
  const uint32_t inv = 0x80000000u / (total > 1u ? total : 1u);  // 2^31 / total (golden.py:174)
  const uint32_t cap = (1u << p.pb) - 1u;
  const int shp = 31 - p.pb;
  const uint64_t pc = 1ull << (shp - 1);
  const bool three = p.pb > 14;
  v4i sel[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t bit = lg == e ? 1u << (8 * (lr & 3)) : 0u;
    sel[e] = v4i{(lr >> 2) == 0 ? (int)bit : 0, (lr >> 2) == 1 ? (int)bit : 0, (lr >> 2) == 2 ? (int)bit : 0,
                 (lr >> 2) == 3 ? (int)bit : 0};
  }
  v4i oacc[DB];
#pragma unroll
  for (int e = 0; e < DB; ++e) oacc[e] = v4i{0, 0, 0, 0};
  for (int kt = kt0 + wave; kt < kt1; kt += nw) {
    v4i vf[4][DK];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int c = 0; c < DK; ++c) vf[b][c] = ld16(vr, frag_off(kt, b, c));
    v4i st[4];
    scores(kt, st);
    v4i pd[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t pn[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t pr = key(kt, j, r) < tlim ? prob_lds(mx - st[j][r], pq, ei, ef) : 0u;
        const uint32_t v = (uint32_t)(((uint64_t)pr * inv + pc) >> shp);
        pn[r] = v < cap ? v : cap;
      }
      pd[0][j] = (int)pack4(pn[0] & 127, pn[1] & 127, pn[2] & 127, pn[3] & 127);
      pd[1][j] = (int)pack4((pn[0] >> 7) & 127, (pn[1] >> 7) & 127, (pn[2] >> 7) & 127, (pn[3] >> 7) & 127);
      pd[2][j] = (int)pack4(pn[0] >> 14, pn[1] >> 14, pn[2] >> 14, pn[3] >> 14);
    }
#pragma unroll
    for (int e = 0; e < DB; ++e) {
      const int c = e >> 2;
      v4i vt;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const v4i t = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf[b][c], sel[e & 3], v4i{0, 0, 0, 0}, 0, 0, 0);
        vt[b] = (int)pack4(t[0], t[1], t[2], t[3]);
      }
      const v4i a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(pd[0], vt, v4i{0, 0, 0, 0}, 0, 0, 0);
      const v4i a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(pd[1], vt, v4i{0, 0, 0, 0}, 0, 0, 0);
      const v4i a2 = three ? __builtin_amdgcn_mfma_i32_16x16x64_i8(pd[2], vt, v4i{0, 0, 0, 0}, 0, 0, 0) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; ++r) oacc[e][r] += a0[r] + 128 * a1[r] + 16384 * a2[r];
    }
  }
#pragma unroll
  for (int e = 0; e < DB; ++e)
#pragma unroll
    for (int r = 0; r < 4; ++r) atomicAdd(&osum[PHASE == 3 ? 4 * lg + r : 0][PHASE == 3 ? 16 * e + lr : 0], oacc[e][r]);
  __syncthreads();
  // the block's valid rows only (the finishing kernel reads no others)
  int32_t* dst = w.outv + (pair * S + z) * AT_ROWS * D;
  const int nrows = min(AT_ROWS, p.M - m0);
  for (int idx = tid; idx < nrows * D; idx += blockDim.x) dst[idx] = (&osum[0][0])[idx];
}

// sum of the S value partials of each (row block, head) pair, then the output requant: one
// thread per output element (grid z covers the block's rows in groups of 256 / D)
template <int D>
__global__ __launch_bounds__(256) void attention_split_finish(AttnArgs p, int S, const int32_t* ws) {
  const int h = blockIdx.x, rb = blockIdx.y;
  const int64_t pairs = (int64_t)p.H * gridDim.y;
  const int64_t pair = (int64_t)h * gridDim.y + rb;
  const int32_t* outv = ws + 2 * pairs * S * AT_ROWS + pair * S * AT_ROWS * D;
  const int idx = (int)blockIdx.z * 256 + (int)threadIdx.x;
  const int row = idx / D, d = idx % D;
  if (row >= AT_ROWS || rb * AT_ROWS + row >= p.M) return;
  int32_t o = 0;
#pragma unroll 8
  for (int q = 0; q < S; ++q) o += outv[(int64_t)q * AT_ROWS * D + idx];
  if (p.pb == 15) o = rshr32(o, 7);
  p.out[(int64_t)(rb * AT_ROWS + row) * p.ldo + (int64_t)h * D + d] = (int8_t)sat8(mulshift(o, p.Mo, p.So));
}

// split-context finish of one row with the output projection: workgroup h sums the S value
// partials of head h, requantises the head's D outputs, then adds its output-projection partial sums
// The output projection's columns are split over gridDim.y workgroups per head (WO_SLICE columns each):
// every workgroup of head h sums the partials and requantises (one of them stores the outputs), then
// adds the partial sums of its columns.
constexpr int WO_SLICE = 128;

template <int D>
__global__ __launch_bounds__(256) void attention_split_finish_wo(AttnArgs p, int S, const int32_t* ws) {
  __shared__ __attribute__((aligned(16))) int8_t ah[D];
  // the output-projection panel chunks of this thread, requested first: they overlap the partial sums
  constexpr int WPF = (WO_SLICE * (D / 16)) / 256 > 0 ? (WO_SLICE * (D / 16)) / 256 : 1;
  const int h = blockIdx.x, n_lo = (int)blockIdx.y * WO_SLICE, n_hi = min(n_lo + WO_SLICE, p.wo_N);
  v4i wpre[WPF];
  wo_prefetch<D, WPF>(p, h, wpre, n_lo, n_hi);
  const int64_t pairs = p.H;
  const int32_t* outv = ws + 2 * pairs * S * AT_ROWS + (int64_t)h * S * AT_ROWS * D;
  if (h == 0 && blockIdx.y == 0) zero_words(p.zero, p.zero_n);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    int32_t o = 0;
    for (int q = 0; q < S; ++q) o += outv[(int64_t)q * AT_ROWS * D + d];
    if (p.pb == 15) o = rshr32(o, 7);
    const int8_t y = (int8_t)sat8(mulshift(o, p.Mo, p.So));
    if (blockIdx.y == 0) p.out[(int64_t)h * D + d] = y;
    ah[d] = y;
  }
  __syncthreads();
  wo_partial<D, WPF>(p, h, ah, wpre, n_lo, n_hi);
}

// ---------------------------------------------------------------------------------------
// attention_row_fused: one row's attention over a long context and the output projection's partial
// sums in ONE launch (the decode chain, one query row).  Grid H x S: workgroup (h, z) takes keys
// [z Tz, (z + 1) Tz) of head h.  The three global reductions of golden.py:167-177 (max, sum of the
// LUT exponentials, probability-weighted value sums) are exchanged between the S workgroups of a
// head through tagged 64-bit words in `st` (the launch's tag in the high half, the value in the
// low half: a reader that sees the tag sees the value, one trip through memory), each wait
// bounded.  Then every workgroup of the head sums the S partials of its D dimensions and
// requantises them, and workgroup z adds the products with output-projection columns
// [z N / S, (z + 1) N / S) into the accumulators: one add per column and head (with one per column
// and workgroup, 256-way contention on each column's word cost microseconds).  Every partial is an
// exact integer max or sum: the split changes no result.
// The S workgroups of a head wait for each other, so the grid (H x S <= CUs) must be resident at
// once; workgroup b = h + H z runs on XCD b % 8, so with H a multiple of 8 a head's workgroups
// share one XCD.  `st`: [0] launches, [1] workgroups done, [2] error, [3] abort, then from word 64
// the exchange words [H][S][2 + D] (uint64: max, sum, D value partials).
// ---------------------------------------------------------------------------------------
constexpr int ARF_THREADS = 256;
constexpr uint32_t ARF_SPIN = 1u << 20;

// the tagged word of `tag` at p (one 8-byte load a pass), or false on timeout / abort
__device__ __forceinline__ bool arf_take(Rsrc r, uint32_t off, uint32_t tag, uint32_t* st, int32_t& v) {
  const Rsrc cr = rsrc(st, 16);
  for (uint32_t it = 0;; ++it) {
    __asm__ volatile("" ::: "memory");  // a fresh load on every pass
    const v2i w = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16));
    if ((uint32_t)w.y == tag) {
      v = w.x;
      return true;
    }
    if (it >= ARF_SPIN) {
      __hip_atomic_fetch_or(st + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(st + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((it & 31) == 31 && __builtin_amdgcn_raw_buffer_load_b32(cr, 12, 0, 16) != 0) return false;
  }
}
// the tagged words at offsets off[0..8) (LD_OOB: none), all eight loads in flight per pass, until
// every one carries `tag`; false on timeout / abort
__device__ __forceinline__ bool arf_take8(Rsrc r, const uint32_t* off, uint32_t tag, uint32_t* st, int32_t* v) {
  const Rsrc cr = rsrc(st, 16);
  for (uint32_t it = 0;; ++it) {
    __asm__ volatile("" ::: "memory");  // fresh loads on every pass
    v2i w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r, off[k], 0, 16));
    bool ok = true;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      ok = ok && (off[k] == LD_OOB || (uint32_t)w[k].y == tag);
      v[k] = w[k].x;
    }
    if (ok) return true;
    if (it >= ARF_SPIN) {
      __hip_atomic_fetch_or(st + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(st + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((it & 31) == 31 && __builtin_amdgcn_raw_buffer_load_b32(cr, 12, 0, 16) != 0) return false;
  }
}
__device__ __forceinline__ void arf_put(Rsrc r, uint32_t off, uint32_t tag, int32_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2i, v2i{v, (int32_t)tag}), r, off, 0, 16);
}

template <int D, int NK>
__global__ __launch_bounds__(ARF_THREADS) void attention_row_fused(AttnArgs p, int S, uint32_t* st) {
  constexpr int CH = D / 16;              // threads per key (16-byte chunks)
  constexpr int KP = ARF_THREADS / CH;    // keys per pass
  __shared__ uint32_t lut32[LUT_DW];
  __shared__ int32_t red[4];
  __shared__ int32_t bc;
  __shared__ int32_t part[KP][D + 1];
  __shared__ __attribute__((aligned(16))) int8_t ah[D];
  __shared__ int ok_s;
  const int h = (int)blockIdx.x, z = (int)blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = tid % CH, k0 = tid / CH;
  const int G = p.H / p.Hkv, g = h / G;
  const int DS = D / S;
  const Rsrc sr = rsrc(st, 16);
  const uint32_t tag = __builtin_amdgcn_raw_buffer_load_b32(sr, 0, 0, 16) + 1u;  // this launch's tag
  if (__builtin_amdgcn_raw_buffer_load_b32(sr, 12, 0, 16) != 0) return;  // an earlier launch gave up (sticky)
  const Rsrc xr = rsrc(st + 64, (int64_t)p.H * S * (2 + D) * 8);
  auto word = [&](int zz, int i) { return (uint32_t)(((h * S + zz) * (2 + D) + i) * 8); };
  const int pos = load_pos(p.pos_dev, p.pos);
  const int T = min(pos + 1, (int)p.max_seq);
  const int Tz = (T + S - 1) / S, t0 = z * Tz, t1 = min(T, t0 + Tz);
  const int8_t* kbase = p.kc + (int64_t)g * p.max_seq * D;
  const int8_t* vbase = p.vc + (int64_t)g * p.max_seq * D;
  const Rsrc kr = rsrc(kbase, (int64_t)T * D), vr = rsrc(vbase, (int64_t)T * D);

  // loads in order of use: q chunk, this thread's key chunks, the LUT, its value chunks
  const v4i qv = ld16(rsrc(p.q + (int64_t)h * D, D), 16u * kc);
  v4i kreg[NK], vreg[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int t = t0 + k0 + KP * i;
    kreg[i] = ld16(kr, t < t1 ? (uint32_t)(t * D + 16 * kc) : LD_OOB);
  }
  if (wave == 0) {
    const Rsrc ir = rsrc(kExpI, sizeof(kExpI)), fr = rsrc(kExpF, sizeof(kExpF));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int idx = lane + 64 * i;
      const uint32_t lw = (uint32_t)ld4(ir, idx < 8 ? 4 * idx : LD_OOB) |
                          (uint32_t)ld4(fr, idx >= 8 && idx < LUT_DW ? 4 * (idx - 8) : LD_OOB);
      if (idx < LUT_DW) lut32[idx] = lw;
    }
  }
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int t = t0 + k0 + KP * i;
    vreg[i] = ld16(vr, t < t1 ? (uint32_t)(t * D + 16 * kc) : LD_OOB);
  }
  // this workgroup's output-projection columns [z NS, z NS + NS), the first 2 KP of them requested
  // now (they do not depend on the attention)
  const int NS = (p.wo_N + S - 1) / S, n_lo = z * NS, n_hi = min(p.wo_N, n_lo + NS);
  const Rsrc wr = rsrc(p.wop + (int64_t)h * p.wo_N * D, (int64_t)p.wo_N * D);
  v4i wpre[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int n = n_lo + u * KP + k0;
    wpre[u] = ld16(wr, n < n_hi ? (uint32_t)(n * D + 16 * kc) : LD_OOB);
  }
  if (h == 0 && z == 0) zero_words(p.zero, p.zero_n);

  // scores and this split's maximum
  int32_t sreg[NK];
  int32_t lmax = INT32_MIN;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    sreg[i] = chunk_sum<CH>(dot16(qv, kreg[i]));
    if (t0 + k0 + KP * i < t1) lmax = max(lmax, sreg[i]);
  }
  lmax = wave_max_i32(lmax);
  if (lane == 0) red[wave] = lmax;
  __syncthreads();
  if (tid == 0) arf_put(xr, word(z, 0), tag, max(max(red[0], red[1]), max(red[2], red[3])));
  // the head's maximum over its S splits
  if (wave == 0) {
    int32_t v = INT32_MIN;
    bool ok = true;
    if (lane < S) ok = arf_take(xr, word(lane, 0), tag, st, v);
    v = wave_max_i32(v);
    const bool all = __builtin_amdgcn_ballot_w64(!ok) == 0;
    if (lane == 0) {
      bc = v;
      ok_s = all;
    }
  }
  __syncthreads();
  if (!ok_s) return;
  const int32_t mx = bc;
  const uint16_t* ei = reinterpret_cast<const uint16_t*>(lut32);
  const uint16_t* ef = ei + 16;
  uint32_t pr[NK];
  uint32_t lsum = 0;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    pr[i] = t0 + k0 + KP * i < t1 ? lut_prob_lds(mulshift((int64_t)mx - sreg[i], p.Ms, p.Ss), ei, ef) : 0u;
    if (kc == 0) lsum += pr[i];
  }
  lsum = (uint32_t)wave_sum_i32((int)lsum);  // T * 65535 < 2^31
  __syncthreads();  // every lane read bc and red before they are reused
  if (lane == 0) red[wave] = (int32_t)lsum;
  __syncthreads();
  if (tid == 0) arf_put(xr, word(z, 1), tag, red[0] + red[1] + red[2] + red[3]);
  if (wave == 0) {
    int32_t v = 0;
    bool ok = true;
    if (lane < S) ok = arf_take(xr, word(lane, 1), tag, st, v);
    v = wave_sum_i32(v);
    const bool all = __builtin_amdgcn_ballot_w64(!ok) == 0;
    if (lane == 0) {
      bc = v;
      ok_s = all;
    }
  }
  __syncthreads();
  if (!ok_s) return;
  const uint32_t total = (uint32_t)bc;
  const uint32_t inv = 0x80000000u / (total > 1u ? total : 1u);  // 2^31 / total (golden.py:174)
  const int32_t cap = (1 << p.pb) - 1;
  const int shp = 31 - p.pb;
  // this split's value sums: 16 dimensions (chunk kc) of this thread's keys, then over the key groups
  int32_t o[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) o[j] = 0;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int64_t q = rshr((int64_t)pr[i] * (int64_t)inv, shp);
    const int32_t pn = (int32_t)(q < cap ? q : cap);
#pragma unroll
    for (int j = 0; j < 16; ++j) o[j] += pn * (int32_t)(int8_t)((uint32_t)vreg[i][j >> 2] >> (8 * (j & 3)));
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) part[k0][16 * kc + j] = o[j];
  __syncthreads();
  if (tid < D) {
    int32_t sum = 0;
    for (int r = 0; r < KP; ++r) sum += part[r][tid];
    arf_put(xr, word(z, 2 + tid), tag, sum);
  }
  // the head's D outputs: every workgroup sums the S partials of every dimension (S D tagged words,
  // eight loads in flight per thread) and requantises them (golden.py:175-180)
  __syncthreads();  // part is reused below
  {
    uint32_t off[8];
    int32_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int f = tid + ARF_THREADS * k;  // word (f / D, f % D)
      off[k] = f < S * D ? word(f / D, 2 + f % D) : LD_OOB;
    }
    const bool ok = arf_take8(xr, off, tag, st, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int f = tid + ARF_THREADS * k;
      if (f < S * D) part[f / D][f % D] = v[k];
    }
    if (!ok) ok_s = 0;
  }
  __syncthreads();
  if (!ok_s) return;
  if (tid < D) {
    int32_t ov = 0;
    for (int zz = 0; zz < S; ++zz) ov += part[zz][tid];
    if (p.pb == 15) ov = rshr32(ov, 7);
    const int8_t y = (int8_t)sat8(mulshift(ov, p.Mo, p.So));
    ah[tid] = y;
    if (tid / DS == z) p.out[(int64_t)h * D + tid] = y;  // each workgroup stores its DS of them
  }
  __syncthreads();
  // the output projection's partial sums of head h for columns [z NS, z NS + NS): CH lanes per column
  // (16-byte chunks of the panel row [h][n][:]), their products summed within the lanes' group, one
  // device-scope add per column (each column gets one add per head, not one per workgroup)
  {
    const v4i a = *reinterpret_cast<const v4i*>(ah + 16 * kc);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int n = n_lo + u * KP + k0;
      const int32_t sacc = chunk_sum<CH>(dot16(a, wpre[u]));
      if (kc == 0 && n < n_hi && sacc != 0) atomic_add_dev(p.wo_acc + n, sacc);
    }
    for (int n0 = n_lo + 2 * KP; n0 < n_hi; n0 += 4 * KP) {
      v4i w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int n = n0 + u * KP + k0;
        w[u] = ld16(wr, n < n_hi ? (uint32_t)(n * D + 16 * kc) : LD_OOB);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int n = n0 + u * KP + k0;
        const int32_t sacc = chunk_sum<CH>(dot16(a, w[u]));
        if (kc == 0 && n < n_hi && sacc != 0) atomic_add_dev(p.wo_acc + n, sacc);
      }
    }
  }
  // launch count: the last workgroup to finish advances the tag of the next launch
  __syncthreads();
  if (tid == 0) {
    const uint32_t done = __hip_atomic_fetch_add(st + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == (uint32_t)(gridDim.x * gridDim.y) - 1u) {
      __hip_atomic_store(st + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(st + 0, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

__global__ void kv_write_kernel(const int8_t* __restrict__ k, const int8_t* __restrict__ v, int64_t M, int Hkv, int D,
                                int64_t ldk, int64_t ldv, int pos, const int32_t* __restrict__ pos_dev,
                                const int32_t* __restrict__ row_pos, int64_t slot_stride, int8_t* __restrict__ kc,
                                int8_t* __restrict__ vc, int64_t max_seq) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = (int64_t)Hkv * D;
  if (idx >= M * per_row) return;
  const int64_t m = idx / per_row;
  const int rem = (int)(idx % per_row);
  const int h = rem / D, d = rem % D;
  const int64_t pm = row_pos ? (int64_t)row_pos[m] : (int64_t)load_pos(pos_dev, pos) + m;
  if (pm < 0 || pm >= max_seq) return;  // device positions are checked by the caller; never write past a cache
  const int64_t dst = (row_pos ? m * slot_stride : 0) + ((int64_t)h * max_seq + pm) * D + d;
  kc[dst] = k[m * ldk + rem];
  vc[dst] = v[m * ldv + rem];
}

}  // namespace llhip

using namespace llhip;

extern "C" {

int llhip_kv_write(const int8_t* k, const int8_t* v, int64_t M, int64_t Hkv, int64_t D, int64_t ldk, int64_t ldv,
                   int64_t pos, const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, int8_t* kc,
                   int8_t* vc, int64_t max_seq, void* stream) {
  if (M < 0 || Hkv <= 0 || D <= 0) return fail(-EINVAL, "kv_write: bad geometry");
  if (ldk < Hkv * D || ldv < Hkv * D) return fail(-EINVAL, "kv_write: leading dimension too small");
  if (row_pos && slot_stride < Hkv * max_seq * D) return fail(-EINVAL, "kv_write: cache slots overlap");
  if (!pos_dev && !row_pos && (pos < 0 || pos + M > max_seq))
    return fail(-ERANGE, "positions %lld..%lld exceed max_seq=%lld", (long long)pos, (long long)(pos + M - 1),
                (long long)max_seq);
  const int64_t total = M * Hkv * D;
  if (total == 0) return 0;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, k, v, M,
                     (int)Hkv, (int)D, ldk, ldv, (int)pos, pos_dev, row_pos, slot_stride, kc, vc, max_seq);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

}  // extern "C"

namespace llhip {

// llhip_attention with the split-context partials in `split_ws` (split_bytes long; NULL disables
// the split): the launch plan is the same for both entry points, except that a plan whose
// partials would not fit takes fewer key splits, or none.
// The output projection folded into a one-row launch (decode chain): panel, accumulators, rows to clear.
struct WoFold {
  const int8_t* wop;
  int32_t* acc;
  int32_t* zero;
  int64_t N, zero_n;
  uint32_t* st;       // attention_row_fused's state (zero-filled once), or null
  int64_t st_bytes;
};

static int attention_impl(const int8_t* q, int64_t M, int64_t H, int64_t Hkv, int64_t D, int64_t ldq, int64_t pos,
                          const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, const int8_t* kc,
                          const int8_t* vc, int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So,
                          int64_t prob_bits, int8_t* out, int64_t ldo, void* split_ws, int64_t split_bytes,
                          void* stream, const WoFold* fold = nullptr, int64_t seq_rows = 0) {
  if (prob_bits != 8 && prob_bits != 15) return fail(-EINVAL, "attention prob_bits must be 8 or 15");
  if (M < 0 || H <= 0 || Hkv <= 0 || H % Hkv) return fail(-EINVAL, "attention: H must be a multiple of Hkv");
  if (D != 16 && D != 32 && D != 64 && D != 128 && D != 256)
    return fail(-EINVAL, "attention: head_dim %lld not in {16,32,64,128,256}", (long long)D);
  if (!u32_ok(Ms) || !u32_ok(Mo) || !shift_ok(Ss) || !shift_ok(So))
    return fail(-EINVAL, "attention: multipliers must be u32, shifts in [0,63]");
  if (ldq < H * D || ldo < H * D) return fail(-EINVAL, "attention: leading dimension too small");
  if (row_pos && slot_stride < Hkv * max_seq * D) return fail(-EINVAL, "attention: cache slots overlap");
  if (seq_rows > 0) {  // sequence-major rows: row m is row m % seq_rows of sequence m / seq_rows
    if (row_pos || pos_dev || fold || seq_rows % AT_ROWS || M % seq_rows)
      return fail(-EINVAL, "attention: sequences of seq_rows rows need M %% seq_rows == 0, seq_rows %% %d == 0",
                  AT_ROWS);
    if (pos < 0 || pos + seq_rows > max_seq)
      return fail(-ERANGE, "positions %lld..%lld exceed max_seq=%lld", (long long)pos,
                  (long long)(pos + seq_rows - 1), (long long)max_seq);
    if (slot_stride < Hkv * max_seq * D) return fail(-EINVAL, "attention: cache slots overlap");
    if (M / seq_rows * slot_stride >= (1ll << 40)) return fail(-EINVAL, "attention: caches too large");
  } else if (!pos_dev && !row_pos && (pos < 0 || pos + M > max_seq)) {
    return fail(-ERANGE, "positions %lld..%lld exceed max_seq=%lld", (long long)pos, (long long)(pos + M - 1),
                (long long)max_seq);
  }
  if (M == 0) return 0;
  const int64_t tmax = (pos_dev || row_pos) ? max_seq : pos + (seq_rows > 0 ? seq_rows : M);
  const bool tiled = !row_pos && (M >= AT_MIN_M || seq_rows > 0);
  if (tmax > (tiled ? AT_MAX_T : ATTN_MAX_T))
    return fail(-EINVAL, "attention: context %lld exceeds %d", (long long)tmax, tiled ? AT_MAX_T : ATTN_MAX_T);
  if (max_seq * D * Hkv >= (1ll << 31)) return fail(-EINVAL, "attention: KV cache above 2 GiB");
  AttnArgs p{};
  p.q = q;
  p.kc = kc;
  p.vc = vc;
  p.out = out;
  p.pos_dev = pos_dev;
  p.row_pos = row_pos;
  p.slot_stride = slot_stride;
  p.seq_rows = (int)seq_rows;
  p.ldq = ldq;
  p.ldo = ldo;
  p.max_seq = max_seq;
  p.Ms = Ms;
  p.Mo = Mo;
  p.Ss = (int)Ss;
  p.So = (int)So;
  p.H = (int)H;
  p.Hkv = (int)Hkv;
  p.pos = (int)pos;
  p.pb = (int)prob_bits;
  p.lds_T = (int)((tmax + 3) / 4 * 4);
  p.M = (int)M;
  if (fold) {
    if (M != 1 || row_pos) return fail(-EINVAL, "dec_attention: one row, one sequence");
    if (!fold->wop || !fold->acc || fold->N < 1 || fold->N > INT32_MAX / D || (uintptr_t)fold->wop % 16 ||
        fold->zero_n < 0 || fold->zero_n > INT32_MAX || (fold->zero_n && !fold->zero) || (uintptr_t)fold->zero % 16)
      return fail(-EINVAL, "dec_attention: bad output-projection panel or accumulators");
    if (H * fold->N * D >= (1ll << 31)) return fail(-EINVAL, "dec_attention: panel above 2 GiB");
    p.wop = fold->wop;
    p.wo_acc = fold->acc;
    p.wo_N = (int)fold->N;
    p.zero = fold->zero;
    p.zero_n = (int)fold->zero_n;
  }
  hipStream_t s = (hipStream_t)stream;
  const int cus = current_cu_count();
  // Long contexts with few (row block, head) pairs: split the key tiles over S workgroups per pair
  // (three reduction launches + a finishing one) so every CU streams a share of K and V.
  const int64_t rblocks = ceil_div(M, AT_ROWS), pairs = H * rblocks, ktiles = ceil_div(tmax, 64);
  // bytes of the partials of S splits: per-split row maxima and sums, and value partials (+ one
  // row's scores for a single-row launch)
  const bool one = M == 1;
  // one row folded into the output projection over a long context: the fused single launch when
  // the caller gave it state and the grid fits the CUs (its workgroups wait for each other)
  if (fold && fold->st && one && !row_pos && (D == 64 || D == 128) && tmax <= AT_MAX_T && ktiles >= AT_SPLIT_MIN_TILES) {
    int S = 16;
    while (S > D / 16 && H * S > cus) S /= 2;
    const int64_t Tz = ceil_div(tmax, S), KP = ARF_THREADS / (D / 16);
    const int64_t nk = ceil_div(Tz, KP);
    const int64_t st_need = 256 + H * S * (2 + D) * 8;
    if (H * S <= cus && nk <= 16 && fold->st_bytes >= st_need && (uintptr_t)fold->st % 16 == 0) {
      dim3 grid((unsigned)H, (unsigned)S), block(ARF_THREADS);
      uint32_t* st = fold->st;
#define LLHIP_ARF(DD)                                                                                   \
  if (nk <= 4) hipLaunchKernelGGL((attention_row_fused<DD, 4>), grid, block, 0, s, p, S, st);          \
  else if (nk <= 8) hipLaunchKernelGGL((attention_row_fused<DD, 8>), grid, block, 0, s, p, S, st);     \
  else hipLaunchKernelGGL((attention_row_fused<DD, 16>), grid, block, 0, s, p, S, st);
      if (D == 64) {
        LLHIP_ARF(64)
      } else {
        LLHIP_ARF(128)
      }
#undef LLHIP_ARF
      LLHIP_LAUNCH_CHECK();
      return 0;
    }
  }
  auto split_need = [&](int64_t S) { return pairs * S * AT_ROWS * (2 + D) * 4 + (one ? pairs * ktiles * 64 * 4 : 0); };
  if (!row_pos && seq_rows == 0 && split_ws && tmax <= AT_MAX_T && ktiles >= AT_SPLIT_MIN_TILES && pairs * 4 <= cus &&
      split_need(2) <= split_bytes) {
    int S = (int)std::min<int64_t>(std::min<int64_t>(ceil_div(cus, pairs), ceil_div(ktiles, 4)), AT_SPLIT_MAXS);
    while (S > 2 && split_need(S) > split_bytes) --S;
    const int tps = (int)ceil_div(ktiles, S);
    S = (int)ceil_div(ktiles, tps);  // never more than before: the plan still fits
    if (split_need(S) > split_bytes) return fail(-EINVAL, "attention: split partials exceed the scratch");
    const int maxw = D <= 128 ? AttnTileCfg<128>::MAXW : AttnTileCfg<256>::MAXW;
    const int nw = std::min(maxw, tps);
    int32_t* sw = static_cast<int32_t*>(split_ws);
    dim3 grid((unsigned)H, (unsigned)rblocks, (unsigned)S), block(64 * nw);
    dim3 fgrid((unsigned)H, (unsigned)rblocks, (unsigned)ceil_div(std::min<int64_t>(M, AT_ROWS) * D, 256));
#define LLHIP_SPLIT(DD)                                                                      \
  if (one) {                                                                                \
    hipLaunchKernelGGL((attention_split<DD, 1, true>), grid, block, 0, s, p, S, tps, sw);   \
    hipLaunchKernelGGL((attention_split<DD, 3, true>), grid, block, 0, s, p, S, tps, sw);   \
  } else {                                                                                  \
    hipLaunchKernelGGL((attention_split<DD, 1, false>), grid, block, 0, s, p, S, tps, sw);  \
    hipLaunchKernelGGL((attention_split<DD, 2, false>), grid, block, 0, s, p, S, tps, sw);  \
    hipLaunchKernelGGL((attention_split<DD, 3, false>), grid, block, 0, s, p, S, tps, sw);  \
  }                                                                                         \
  if (fold)                                                                                 \
    hipLaunchKernelGGL((attention_split_finish_wo<DD>), dim3((unsigned)H, (unsigned)ceil_div(p.wo_N, WO_SLICE)),    \
                       dim3(256), 0, s, p, S, sw);                                                  \
  else                                                                                      \
    hipLaunchKernelGGL((attention_split_finish<DD>), fgrid, dim3(256), 0, s, p, S, sw);
    switch (D) {
      case 16: LLHIP_SPLIT(16) break;
      case 32: LLHIP_SPLIT(32) break;
      case 64: LLHIP_SPLIT(64) break;
      case 128: LLHIP_SPLIT(128) break;
      default: LLHIP_SPLIT(256) break;
    }
#undef LLHIP_SPLIT
    LLHIP_LAUNCH_CHECK();
    return 0;
  }
  if (tiled) {
    // waves per workgroup: enough that every wave's tiles stay in registers across the three
    // passes, more (up to the register-file limit) while the chip would otherwise be idle
    const int64_t blocks = H * ceil_div(M, AT_ROWS);
    const int maxw = D <= 128 ? AttnTileCfg<128>::MAXW : AttnTileCfg<256>::MAXW;
    const int sc = D <= 64 ? AttnTileCfg<64>::SC : 1;
    const int64_t tiles = ceil_div(tmax, 64);
    int nw = 1;
    while (nw < maxw && nw * 2 <= tiles && (nw * sc < tiles || blocks * nw < 4 * (int64_t)current_cu_count())) nw *= 2;
    dim3 grid((unsigned)H, (unsigned)ceil_div(M, AT_ROWS));
    dim3 block(64 * nw);
    const bool dense = blocks * nw > 12ll * current_cu_count();  // more waves than three per SIMD
    switch (D) {
      case 16: hipLaunchKernelGGL(attention_tiled<16>, grid, block, 0, s, p); break;  // 4 waves/SIMD as they are
      case 32: hipLaunchKernelGGL(attention_tiled<32>, grid, block, 0, s, p); break;
      case 64:
        if (dense) hipLaunchKernelGGL((attention_tiled<64, 4>), grid, block, 0, s, p);
        else hipLaunchKernelGGL(attention_tiled<64>, grid, block, 0, s, p);
        break;
      case 128: hipLaunchKernelGGL(attention_tiled<128>, grid, block, 0, s, p); break;
      default: hipLaunchKernelGGL(attention_tiled<256>, grid, block, 0, s, p); break;
    }
    LLHIP_LAUNCH_CHECK();
    return 0;
  }
  const size_t lds = sizeof(int32_t) * (size_t)p.lds_T;
  // the output-projection fold of one row runs D / 16 workgroups per head (dimension slices),
  // heads of D = 256 one workgroup each
  const bool slice = fold && M == 1 && D <= 128;
  const int64_t per_head = slice ? D / 16 : 1;
  if (M * Hkv > (int64_t)INT32_MAX / 8 / (H / Hkv) / per_head) return fail(-EINVAL, "attention: too many rows");
  dim3 grid((unsigned)(8 * ceil_div(M * Hkv, 8) * (H / Hkv) * per_head));
  p.span = 0;
  if (slice && Hkv < 8 && 8 % Hkv == 0) {
    p.span = (int)(8 / Hkv);
    grid = dim3((unsigned)(8 * ceil_div((H / Hkv) * per_head, p.span)));
  }
  dim3 block(ATTN_THREADS);
#define LLHIP_ROWHEAD(DD)                                                            \
  if (slice)                                                                        \
    hipLaunchKernelGGL((attention_rowhead<DD, true, DD <= 128>), grid, block, lds, s, p); \
  else if (fold)                                                                    \
    hipLaunchKernelGGL((attention_rowhead<DD, true>), grid, block, lds, s, p);      \
  else                                                                              \
    hipLaunchKernelGGL((attention_rowhead<DD, false>), grid, block, lds, s, p);
  switch (D) {
    case 16: LLHIP_ROWHEAD(16) break;
    case 32: LLHIP_ROWHEAD(32) break;
    case 64: LLHIP_ROWHEAD(64) break;
    case 128: LLHIP_ROWHEAD(128) break;
    default: LLHIP_ROWHEAD(256) break;
  }
#undef LLHIP_ROWHEAD
  LLHIP_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------------------
// scratch of the allocation-free entry point
// ---------------------------------------------------------------------------------------
// The split-context partials of llhip_attention_noalloc live in this file-scope array: every GPU
// the library runs on holds its own copy until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol): the device address
// comes from hipGetSymbolAddress, once per device with that device current, and is kept below.
constexpr int64_t NOALLOC_SCRATCH_BYTES = (int64_t)LLHIP_ATTENTION_NOALLOC_SCRATCH;
static __device__ __align__(256) int32_t scratch[NOALLOC_SCRATCH_BYTES / 4];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES];

// device address of `scratch` on the current device (looked up on the first call per device)
static int noalloc_scratch(void** out) {
  int dev = 0;
  LLHIP_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(-EINVAL, "attention_noalloc: device %d above %d", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(-EIO, "attention_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace llhip

extern "C" {

int llhip_attention(const int8_t* q, int64_t M, int64_t H, int64_t Hkv, int64_t D, int64_t ldq, int64_t pos,
                    const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, const int8_t* kc,
                    const int8_t* vc, int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So,
                    int64_t prob_bits, int8_t* out, int64_t ldo, void* ws, void* stream) {
  return attention_impl(q, M, H, Hkv, D, ldq, pos, pos_dev, row_pos, slot_stride, kc, vc, max_seq, Ms, Ss, Mo, So,
                        prob_bits, out, ldo, ws ? static_cast<char*>(ws) + WS_SCRATCH : nullptr, WS_SCRATCH_BYTES,
                        stream);
}

int llhip_attention_seqs(const int8_t* q, int64_t M, int64_t seq_rows, int64_t H, int64_t Hkv, int64_t D,
                         int64_t ldq, int64_t pos, const int8_t* kc, const int8_t* vc, int64_t slot_stride,
                         int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So, int64_t prob_bits,
                         int8_t* out, int64_t ldo, void* stream) {
  if (seq_rows <= 0) return fail(-EINVAL, "attention_seqs: seq_rows must be positive");
  return attention_impl(q, M, H, Hkv, D, ldq, pos, nullptr, nullptr, slot_stride, kc, vc, max_seq, Ms, Ss, Mo, So,
                        prob_bits, out, ldo, nullptr, 0, stream, nullptr, seq_rows);
}

int llhip_dec_attention(const llhip_dec_attn_desc* d, void* ws, void* stream) {
  if (!d) return fail(-EINVAL, "dec_attention: null descriptor");
  WoFold f{static_cast<const int8_t*>(d->wo_panel), static_cast<int32_t*>(d->acc), static_cast<int32_t*>(d->zero),
           d->N, d->zero_n, static_cast<uint32_t*>(d->state), d->state_bytes};
  return attention_impl(static_cast<const int8_t*>(d->q), 1, d->H, d->Hkv, d->D, d->H * d->D, d->pos,
                        static_cast<const int32_t*>(d->pos_dev), nullptr, 0, static_cast<const int8_t*>(d->kc),
                        static_cast<const int8_t*>(d->vc), d->max_seq, d->Ms, d->Ss, d->Mo, d->So, d->prob_bits,
                        static_cast<int8_t*>(d->out), d->H * d->D, ws ? static_cast<char*>(ws) + WS_SCRATCH : nullptr,
                        WS_SCRATCH_BYTES, stream, &f);
}

int64_t llhip_dec_attn_state_bytes(int64_t H, int64_t D) {
  if (H < 1 || D < 1 || H > 4096 || D > 256) return fail(-EINVAL, "dec_attn_state_bytes: bad shape");
  return 256 + H * 16 * (2 + D) * 8;
}

int llhip_dec_attn_status(const void* state, int64_t* launches, int64_t* err) {
  if (!state) return fail(-EINVAL, "dec_attn_status: null state");
  uint32_t h[4];
  LLHIP_CHECK_HIP(hipDeviceSynchronize());
  LLHIP_CHECK_HIP(hipMemcpy(h, state, sizeof(h), hipMemcpyDeviceToHost));
  if (launches) *launches = h[0];
  if (err) *err = h[2];
  return 0;
}

int llhip_attention_noalloc(const int8_t* q, int64_t M, int64_t H, int64_t Hkv, int64_t D, int64_t ldq, int64_t pos,
                            const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, const int8_t* kc,
                            const int8_t* vc, int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So,
                            int64_t prob_bits, int8_t* out, int64_t ldo, void* stream) {
  void* sw = nullptr;
  const int rc = noalloc_scratch(&sw);
  if (rc) return rc;
  return attention_impl(q, M, H, Hkv, D, ldq, pos, pos_dev, row_pos, slot_stride, kc, vc, max_seq, Ms, Ss, Mo, So,
                        prob_bits, out, ldo, sw, NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
