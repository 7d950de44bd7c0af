// Decode step of libllhip: every layer of one decode row (golden.py:392-397, which runs the op
// list of golden.py:275-314 for M = 1) in one persistent launch.
//
// Per layer the row passes two stages, each spread over workgroups that own fixed shares:
//   S12 (attention) unit (head h, 16-dimension slice ds), one per workgroup: the layer input row
//        (finished from the previous down projection's int32 partial sums + bias + requant +
//        residual), RMSNorm, quant, then the head's q and its GQA group's k (all D columns) and the
//        slice's 16 v columns, requant, RoPE, quant (golden.py:286-300, 316-342, 141-158), the
//        head's integer softmax over the context with the new key, the slice's 16 outputs, and their
//        exact int32 partial sums of the output projection for every output column (golden.py:
//        162-180, 353-366, 316-342).  Every unit of a group computes the group's new key itself
//        (its q/k weights are read from LDS), so no stage waits for another's q/k/v; the group's
//        first head's units write the new key and values into the KV cache (golden.py:344-351).
//   S3 (mlp) one per remaining workgroup: the output projection finished from those partial sums,
//        RMSNorm, quant, gate (SiLU) and up (mul) for up to two 16-column FFN tiles, quant, and their
//        partial sums of the down projection (golden.py:286-309, 101-107, 316-342).
// Integer sums do not depend on their order, so every value equals the separate ops'.
//
// Hand-offs.  A stage's producers write their results with device-scope stores and atomics, wait
// for them to complete, then store their flag word (the launch's epoch for that layer); the next
// stage's workgroups poll the flags they depend on with device-scope loads and then read the
// results with device-scope loads.  Each workgroup has 8 waves: waves 0-3 (row waves) poll, read
// and finish rows, run the epilogues and issue every store and atomic; waves 4-7 (weight waves)
// hold the stage's weights in LDS, run the projections' MFMAs and request the next layer's weights
// right after their last read, while the row waves wait for other workgroups.  The two sets meet
// through LDS counters, never a workgroup barrier, so a weight wave's run of load issues (paced by
// HBM bandwidth) never holds up a row wave.  The attention runs on all eight waves.
//
// Every wait is bounded (spin_max polls); a timeout records an error word, raises an abort word
// that every other wait also watches, and the workgroup leaves the layer loop, so the launch always
// ends.  The grid is one workgroup per CU (at most 256), all resident at once.
#include <algorithm>
#include <vector>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {
namespace dstep {

constexpr int NTH = 512;    // 4 row waves + 4 weight waves
constexpr int R = 8;        // accumulator replicas: producer j adds into row j % R
constexpr int D = 64;       // head_dim of the decode step
constexpr int DC = D / 16;  // 16-byte chunks per key row
constexpr int KR = 6;       // keys per thread held in registers (512 threads, 4 per key: 768 keys)
constexpr int PNL = 4;      // output-projection / down-projection panel chunks per row thread
constexpr int MAX_DIM = 1024;
constexpr int MAX_G = 256;
constexpr int SC1 = 16;     // buffer cache-policy bit sc1: device-scope coherent access

struct Layer {
  const int16_t* g1;
  const int8_t* W[3];
  const int32_t* rq[3];
  const int32_t* bias[3];
  int8_t* kc;
  int8_t* vc;
  const int8_t* wo;
  const int32_t* rq_o;
  const int32_t* bias_o;
  const int16_t* g2;
  const int8_t* Wg;
  const int8_t* Wu;
  const int32_t* rqg;
  const int32_t* rqu;
  const int32_t* bg;
  const int32_t* bu;
  const int8_t* wd;
  const int32_t* rq_d;
  const int32_t* bias_d;
  int64_t Mq1, Mq2, quant_M[2], Ms, Mo, silu_Mi, fq_M;
  int64_t eps1, C1, eps2, C2;
  int64_t sh1, Sq1, sh2, Sq2, quant_S[2], Ss, So, pb, silu_Si, silu_sh, mul_sh, fq_S;
};

typedef __attribute__((address_space(4))) const Layer CLayer;

struct Args {
  const Layer* layers;
  const int16_t* x_in;
  const int16_t* cos_tab;
  const int16_t* sin_tab;
  const int32_t* pos_dev;
  int16_t* xres;   // [2][dim]: the layer input x, the attention residual x1
  int32_t* acc_o;  // [2][R][dim] output-projection partial sums (layer parity)
  int32_t* acc_d;  // [2][R][dim] down-projection partial sums
  uint32_t* fl0;   // stage flags, [NREP][32 lines][32] words each: S12 units' layer-0 clearing
  uint32_t* fl2;   // S12 units done
  uint32_t* fl3;   // S3 units done
  uint32_t* ctl;   // [0] launches, [1] workgroups done, [2] error, [3] abort
  const int32_t* role;  // [G] workgroup -> S12 unit u (u), S3 unit u (256 + u) or idle (-1)
  uint32_t* kx;         // [H][D] a head's new key (tagged words), exchanged between its slices
  int L, dim, H, Hkv, max_seq, F;
  int nu2, nu3, tiles;  // S12 units (H * D / 16), S3 units with FFN tiles, 16-column FFN tiles
  uint32_t spin_max;
};

// ---- device-scope (coherent) loads and stores -------------------------------------------
__device__ __forceinline__ v4i ldc16(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, SC1));
}
__device__ __forceinline__ v2i ldc8(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, SC1));
}
__device__ __forceinline__ uint32_t ldc4(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, SC1);
}
__device__ __forceinline__ void stc4(Rsrc r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, SC1);
}
__device__ __forceinline__ void stc8(Rsrc r, uint32_t off, v2i v) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), r, off, 0, SC1);
}
// wait for this wave's stores and atomics (and every load) to complete
__device__ __forceinline__ void drain() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// a 1 KiB LDS block at blk (wave-uniform) receives 16 bytes per lane from byte offset off of r, lane
// l at blk + 16 l (direct global-to-LDS load; offsets past the range read zeros)
__device__ __forceinline__ void dma16(Rsrc r, int8_t* blk, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)blk, 16, off, 0, 0, 0);
}
__device__ __forceinline__ v4i lds16(const int8_t* blk) {
  return *reinterpret_cast<const v4i*>(blk + 16 * (threadIdx.x & 63));
}

__device__ __forceinline__ int32_t dot16(const v4i& a, const v4i& b, int32_t s = 0) {
  s = __builtin_amdgcn_sdot4(a.x, b.x, s, false);
  s = __builtin_amdgcn_sdot4(a.y, b.y, s, false);
  s = __builtin_amdgcn_sdot4(a.z, b.z, s, false);
  return __builtin_amdgcn_sdot4(a.w, b.w, s, false);
}
__device__ __forceinline__ int32_t sbyte(int w, int i) { return (int32_t)(int8_t)((uint32_t)w >> (8 * i)); }

// sum over aligned groups of 4 lanes, every lane ending with its group's total
__device__ __forceinline__ int32_t quad_sum(int32_t v) {
  v += dpp_mov<DPP_QUAD_XOR1>(v);
  return v + dpp_mov<DPP_QUAD_XOR2>(v);
}
// sum over the 16 lanes of a row, every lane ending with the row's total
__device__ __forceinline__ int32_t row16_sum(int32_t v) {
  v += dpp_mov<DPP_ROW_ROR + 1>(v);
  v += dpp_mov<DPP_ROW_ROR + 2>(v);
  v += dpp_mov<DPP_ROW_ROR + 4>(v);
  return v + dpp_mov<DPP_ROW_ROR + 8>(v);
}

// Probability of a key whose score lies x below the maximum (golden.py:168-172): z = rshr(x Ms, Ss)
// with x in [0, 2^21] (|score| <= 64 * 128 * 128) and Ms < 2^32 is (x Ms + 2^(Ss-1)) >> Ss, one
// unsigned 32 x 32 + 64 multiply-add and a shift; z >= 4096 is past the exp table (probability 0).
__device__ __forceinline__ uint32_t prob_gap(int32_t x, uint32_t Ms, uint64_t half, int Ss, const uint16_t* ei,
                                             const uint16_t* ef) {
  const uint64_t z = ((uint64_t)(uint32_t)x * Ms + half) >> Ss;
  if (z >= 4096u) return 0u;
  const uint32_t zi = (uint32_t)z;
  return ((uint32_t)ei[zi >> 8] * (uint32_t)ef[zi & 255] + 32768u) >> 16;
}
// Normalised probability min(rshr(p inv, shp), cap) (golden.py:173-176) for p < 2^16, inv <= 2^31,
// shp >= 1: p inv + 2^(shp-1) < 2^48, one multiply-add and a shift.
__device__ __forceinline__ int32_t prob_norm(uint32_t p, uint32_t inv, uint64_t half, int shp, int32_t cap) {
  const uint32_t q = (uint32_t)(((uint64_t)p * inv + half) >> shp);
  return q < (uint32_t)cap ? (int32_t)q : cap;
}

// ---- flags ------------------------------------------------------------------------------------
// Stage flags: each producer writes its word into NREP replicas; workgroup b polls replica b % NREP
// (the replica of its XCD), so no line has more than G / NREP pollers.  Within a replica the n
// producers' words are spread over nl = min(32, ceil(n / 4)) lines of 32 words (word of producer u:
// line u % nl, slot u / nl), so a line takes at most 4 writes at once (8 for 200+ producers): the
// memory side serialises the partial writes to one line, and 56 or 200 of them packed into two or
// seven lines completed up to a microsecond apart from replica to replica (8 writers a line:
// 364 us a step, 4: 361 us, 64 lines of 4: no better).
constexpr int NREP = 8;
constexpr int REP_WORDS = 32 * 32;  // 32 lines of 32 words (4 KiB) per replica
constexpr int FLAG_WORDS = REP_WORDS * NREP;
__device__ __forceinline__ int flag_lines(int n) { return min(32, (n + 3) / 4); }
__device__ __forceinline__ uint32_t flag_off(int u, int nl) { return 4u * (uint32_t)((u % nl) * 32 + u / nl); }

// Wave 0: wait until the words of producers [0, n) (n <= 256) in replica f all reach `want` (signed
// 32-bit difference, so epochs may wrap).  False on timeout (recorded) or abort.  Lane i reads the
// words of producers i, i + 64, i + 128, i + 192.
__device__ bool poll(const uint32_t* f, int n, uint32_t want, uint32_t* ctl, uint32_t spin_max) {
  const int lane = threadIdx.x & 63, nl = flag_lines(n);
  const Rsrc fr = rsrc(f, REP_WORDS * 4), cr = rsrc(ctl, 16);
  uint32_t off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) off[j] = lane + 64 * j < n ? flag_off(lane + 64 * j, nl) : LD_OOB;
  for (uint32_t it = 0;; ++it) {
    __asm__ volatile("" ::: "memory");  // fresh loads on every pass
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = ldc4(fr, off[j]);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) ok = ok && (lane + 64 * j >= n || (int32_t)(v[j] - want) >= 0);
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
    if (it >= spin_max) {
      if (lane == 0) {
        __hip_atomic_fetch_or(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ctl + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return false;
    }
    if ((it & 31) == 31 && ldc4(cr, 12) != 0) return false;  // another workgroup gave up
  }
}

// Tagged words: (tag << 16) | (value & 0xFFFF) in one 32-bit store, so a reader that sees the tag of
// the current layer sees the value with it (no separate flag: one trip through memory).  The wave
// waits until word `lane` of p (D words) carries `tag` and returns its 16-bit value; `first` is a
// load of that word issued earlier (its latency hidden behind other work).  False on timeout
// (recorded) or abort.
__device__ bool take_tagged(const uint32_t* p, uint32_t tag, uint32_t first, uint32_t* ctl, uint32_t spin_max,
                            int32_t& val) {
  const int lane = threadIdx.x & 63;
  if (__builtin_amdgcn_ballot_w64((first >> 16) != tag) == 0) {
    val = (int32_t)(int16_t)(first & 0xFFFFu);
    return true;
  }
  const Rsrc pr = rsrc(p, 4 * D), cr = rsrc(ctl, 16);
  uint32_t nxt = ldc4(pr, 4u * lane);
  for (uint32_t it = 0;; ++it) {
    __asm__ volatile("" ::: "memory");  // a fresh load on every pass
    const uint32_t cur = nxt;
    nxt = ldc4(pr, 4u * lane);
    __asm__ volatile("s_waitcnt vmcnt(1)" ::: "memory");  // cur has arrived, nxt may still be in flight
    if (__builtin_amdgcn_ballot_w64((cur >> 16) != tag) == 0) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      val = (int32_t)(int16_t)(cur & 0xFFFFu);
      return true;
    }
    if (it >= spin_max) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lane == 0) {
        __hip_atomic_fetch_or(ctl + 2, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ctl + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return false;
    }
    if ((it & 31) == 31 && ldc4(cr, 12) != 0) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      return false;
    }
  }
}

// wave 0: store the flag word of producer idx into every replica (after the workgroup's drain)
__device__ __forceinline__ void publish(uint32_t* f, int idx, int n, uint32_t v) {
  const int lane = threadIdx.x & 63;
  if (lane < NREP) stc4(rsrc(f, FLAG_WORDS * 4), 4u * REP_WORDS * lane + flag_off(idx, flag_lines(n)), v);
}

// ---- LDS hand-offs inside the workgroup ------------------------------------------------------
// Monotonic LDS counters: a wave's LDS writes complete, then its lane 0 adds one; a reader waits
// until the count reaches its target.  The abort word ends every wait when the launch is being
// abandoned.
struct Sync {
  uint32_t rowbar, allbar, xrdy, wrdy, krdy, aiss, abort;  // krdy: k partials in; aiss: flag published
};

__device__ __forceinline__ void sig_add(uint32_t* c) {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// false when the abort word is set
__device__ __forceinline__ bool sig_wait(uint32_t* c, uint32_t target, uint32_t* abortp) {
  while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    if (__hip_atomic_load(abortp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  __asm__ volatile("" ::: "memory");  // LDS reads of the other waves' values stay after the wait
  return true;
}

// ---- row-wave helpers (row thread rt owns elements 4rt..4rt+3) ---------------------------------
struct RowOps {
  v4i rq0, rq1, bias;  // requant pairs and bias of the projection finished into this row
  v2i g;               // RMSNorm gamma
};

__device__ __forceinline__ void rowops_load(RowOps& o, const int32_t* rq, const int32_t* bias, const int16_t* g,
                                            int dim, int rt) {
  const bool in = 4 * rt < dim;
  const Rsrc qr = rsrc(rq, (int64_t)dim * 8);
  o.rq0 = ld16(qr, in ? 32u * rt : LD_OOB);
  o.rq1 = ld16(qr, in ? 32u * rt + 16u : LD_OOB);
  o.bias = ld16(rsrc(bias, (int64_t)dim * 4), in ? 16u * rt : LD_OOB);
  o.g = ld8(rsrc(g, (int64_t)dim * 2), in ? 8u * rt : LD_OOB);
}

// x[j] = sat16(sat16(mulshift(sum_r acc[r][n] + bias[n], M_n, S_n)) + aux[n]) (golden.py:324-336,
// resadd) for n = 4rt + j; acc and aux were written in this launch (device-scope loads)
__device__ __forceinline__ void finish4(const int32_t* acc, const int16_t* aux, const RowOps& o, int dim, int rt,
                                        int32_t x[4]) {
  const bool in = 4 * rt < dim;
  const Rsrc ar = rsrc(acc, (int64_t)R * dim * 4);
  v4i s[R];
#pragma unroll
  for (int r = 0; r < R; ++r) s[r] = ldc16(ar, in ? (uint32_t)((r * dim + 4 * rt) * 4) : LD_OOB);
  const v2i xa = ldc8(rsrc(aux, (int64_t)dim * 2), in ? 8u * rt : LD_OOB);
  const int32_t xv[4] = {lo16(xa.x), hi16(xa.x), lo16(xa.y), hi16(xa.y)};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int32_t t = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) t += s[r][j];
    const int32_t M = j < 2 ? o.rq0[2 * j] : o.rq1[2 * (j - 2)];
    const int32_t S = j < 2 ? o.rq0[2 * j + 1] : o.rq1[2 * (j - 2) + 1];
    const int64_t v = sat16(mulshift((int64_t)t + o.bias[j], (int64_t)M, S));
    x[j] = (int32_t)sat16(v + xv[j]);
  }
}

// clear words [lo, hi) of the two accumulator blocks of parity par (acc_o then acc_d, R*dim each)
__device__ __forceinline__ void zero_slice(const Args& a, int par, int lo, int hi, int rt) {
  const int n = R * a.dim;
  const Rsrc o = rsrc(a.acc_o + (int64_t)par * n, (int64_t)n * 4), d = rsrc(a.acc_d + (int64_t)par * n, (int64_t)n * 4);
  for (int i = lo + rt; i < hi; i += 256) {
    if (i < n) stc4(o, 4u * i, 0u);
    else stc4(d, 4u * (i - n), 0u);
  }
}

// LDS of the two kinds of workgroup (dynamic part; the scores follow the blocks).  Each weight wave
// owns 1 KiB blocks (lane l's 16 bytes at 16 l), filled by direct loads in the order it reads them.
//   S12: per weight wave w, q tile w of head h over all K steps, then K steps w VS .. w VS + VS - 1
//        of the slice's k and v tiles: KST + 2 VS blocks.
//   S3 : per weight wave (gate or up, K half), NS3 steps of each of the two FFN tiles: 2 NS3 blocks.
template <int KST>
struct StepCfg {
  static constexpr int VS = (KST + 3) / 4;
  static constexpr int NB12 = KST + 2 * VS;
  static constexpr int NS3 = (KST + 1) / 2;
  static constexpr int NB3 = 2 * NS3;
  static constexpr int NB = NB12 > NB3 ? NB12 : NB3;
  static constexpr int SC_OFF = 4 * NB * 1024;
};

template <int KST>
__global__ __launch_bounds__(NTH) void dec_step_kernel(Args a) {
  kernarg_warm<sizeof(Args)>();
  using C = StepCfg<KST>;
  constexpr int VS = C::VS, NS3 = C::NS3, NB = C::NB;

  __shared__ __attribute__((aligned(16))) int8_t xq[KST * 64 + 16];
  __shared__ __attribute__((aligned(16))) int8_t q8[D];
  __shared__ __attribute__((aligned(16))) int8_t k8[D];
  __shared__ __attribute__((aligned(16))) int8_t vnew[16];
  __shared__ __attribute__((aligned(16))) int8_t ah[16];
  __shared__ __attribute__((aligned(16))) int8_t fq16[2][16];
  __shared__ uint64_t red64[4];
  __shared__ int32_t gq[D], gk[4][16], gv[4][16];  // q; k and v slice: per weight wave K-step partial sums
  __shared__ int32_t yq[D], yk[D];
  __shared__ int32_t redmax[8], redsum[8];
  __shared__ int32_t wpart[32][16];
  __shared__ int32_t red3[2][4][16];
  __shared__ uint32_t lut32[136];
  __shared__ uint32_t sig32[192];
  __shared__ int okw;
  __shared__ Sync sy;
  extern __shared__ __attribute__((aligned(1024))) int8_t dyn[];
  int32_t* sc = reinterpret_cast<int32_t*>(dyn + C::SC_OFF);  // [max_seq] scores, then probabilities

  const int b = blockIdx.x, G = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const bool roww = wave < 4;
  const int rt = tid;   // row thread index (row waves)
  const int w4 = wave - 4;
  const int dim = a.dim;  // 64 KST
  const int role = ((const __attribute__((address_space(4))) int32_t*)a.role)[b];
  const int u2 = role >= 0 && role < 256 ? role : -1;  // S12 unit
  const int u3 = role >= 256 ? role - 256 : -1;        // S3 unit
  const int rep = b % NREP;  // flag replica this workgroup polls
  const int col = lane & 15, kg = lane >> 4;
  const CLayer* lyr = (const CLayer*)a.layers;  // read-only for the launch: scalar loads
  const Rsrc ctlr = rsrc(a.ctl, 16);
  const uint32_t seq = ldc4(ctlr, 0);
  const uint32_t e0 = seq * 64u;
  const int pos = *(const __attribute__((address_space(4))) int32_t*)a.pos_dev;  // written by an earlier launch
  const int T = pos + 1;
  const bool dead0 = ldc4(ctlr, 12) != 0 || pos < 0 || pos >= a.max_seq;
  if (b == 0 && tid == 0 && (pos < 0 || pos >= a.max_seq))  // the caller checks positions; record it anyway
    __hip_atomic_fetch_or(a.ctl + 2, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // S12 geometry: head h, value slice ds, GQA group g; its group's first head writes the cache row
  const int h = u2 >= 0 ? u2 / DC : 0, ds = u2 >= 0 ? u2 % DC : 0;
  const int g = h / (a.H / a.Hkv);
  const bool kv_writer = h % (a.H / a.Hkv) == 0;
  // S3 geometry: FFN tiles ta and tb (tb < 0: one tile)
  const int ta = u3, tb = (u3 >= 0 && u3 + a.nu3 < a.tiles) ? u3 + a.nu3 : -1;

  // ---- constant tables into LDS, zero padding of the quantised row, RoPE factors ----
  int32_t cs = 0, sn = 0;  // lane p < D/2: RoPE pair (p, p + D/2) factors (q: wave 0; new key: any wave)
  if (wave == 0) {
    const Rsrc ir = rsrc(kExpI, sizeof(kExpI)), fr = rsrc(kExpF, sizeof(kExpF)), sr = rsrc(kSig, sizeof(kSig));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int idx = lane + 64 * i;
      const uint32_t lw = (uint32_t)ld4(ir, idx < 8 ? 4 * idx : LD_OOB) |
                          (uint32_t)ld4(fr, idx >= 8 && idx < 136 ? 4 * (idx - 8) : LD_OOB);
      if (idx < 136) lut32[idx] = lw;
      sig32[idx] = (uint32_t)ld4(sr, idx < 129 ? 4 * idx : LD_OOB);
    }
  }
  if (u2 >= 0 && lane < D / 2) {
    const Rsrc cr = rsrc(a.cos_tab, (int64_t)a.max_seq * D), snr = rsrc(a.sin_tab, (int64_t)a.max_seq * D);
    const uint32_t off = dead0 ? LD_OOB : (uint32_t)(((int64_t)pos * (D / 2) + lane) * 2);
    cs = ld2s(cr, off);
    sn = ld2s(snr, off);
  }
  for (int i = dim + tid; i < KST * 64 + 16; i += NTH) xq[i] = 0;  // K steps past the row multiply zeros
  if (!roww) {  // blocks that are never loaded (steps past the row, an absent FFN tile) read as zeros
    int8_t* bw = dyn + (wave - 4) * NB * 1024;
    for (int i = 16 * lane; i < NB * 1024; i += 1024) *reinterpret_cast<v4i*>(bw + i) = v4i{0, 0, 0, 0};
  }
  if (tid == 0) sy = Sync{0u, 0u, 0u, 0u, 0u, 0u, 0u};
  __syncthreads();  // the only workgroup barrier: tables and counters in place

  const uint16_t* ei = reinterpret_cast<const uint16_t*>(lut32);
  const uint16_t* ef = ei + 16;
  const uint16_t* sig = reinterpret_cast<const uint16_t*>(sig32);
  int8_t* blk = dyn + w4 * NB * 1024;  // this weight wave's blocks
  uint32_t nrow = 0, nall = 0, nx = 0, nw = 0, nk = 0;
  bool alive = !dead0 && (u2 >= 0 || u3 >= 0);

  auto row_meet = [&]() -> bool {  // the four row waves
    sig_add(&sy.rowbar);
    nrow += 4;
    return sig_wait(&sy.rowbar, nrow, &sy.abort);
  };
  auto all_meet = [&]() -> bool {  // all eight waves
    sig_add(&sy.allbar);
    nall += 8;
    return sig_wait(&sy.allbar, nall, &sy.abort);
  };
  // row waves, after wave 0 polled: every row wave learns the result
  auto row_polled = [&](bool ok) -> bool {
    if (wave == 0 && lane == 0) okw = ok;
    if (!row_meet()) return false;
    if (!okw) {
      if (lane == 0) __hip_atomic_store(&sy.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      return false;
    }
    return true;
  };
  // RMSNorm (golden.py:124-137) and quant (golden.py:119-120) of the row the row threads hold: the
  // sum of squares over the four row waves (one meeting), then the quantised bytes into xq
  auto norm_quant = [&](const int32_t x[4], const v2i& gm, uint32_t eps, uint32_t Cn, int sh, int64_t Mq,
                        int Sq) -> bool {
    uint64_t ss = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) ss += (uint64_t)(uint32_t)(x[j] * x[j]);
    ss = wave_sum_u64(ss);
    if (lane == 0) red64[wave] = ss;
    if (!row_meet()) return false;
    if (4 * rt < dim) {
      const uint32_t inv = rms_inv(red64[0] + red64[1] + red64[2] + red64[3], eps, Cn);
      const double sy_ = rms_scale(inv, sh), sq = mulshift_scale(Mq, Sq);
      const int32_t gv_[4] = {lo16(gm.x), hi16(gm.x), lo16(gm.y), hi16(gm.y)};
      uint32_t q = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int32_t y = rms_apply_d(x[j], gv_[j], sy_);
        q |= (uint32_t)(uint8_t)mulshift_small_sat(y, sq, -128.0, 127.0) << (8 * j);
      }
      *reinterpret_cast<uint32_t*>(xq + 4 * rt) = q;
    }
    return true;
  };

  if (u2 >= 0) {
    // =============================== S12 unit (h, ds) ===============================
    // Weight wave w: blocks [0, KST) q tile w of head h (all K steps); [KST, KST + VS) and
    // [KST + VS, KST + 2 VS) K steps w VS .. w VS + VS - 1 of the slice's k and v columns
    // 16 ds .. 16 ds + 15 of group g (steps past the row are never loaded: zero).  The head's four
    // slices trade their k columns (the new key is needed last, after the cached keys' scores).
    auto w_issue = [&](const CLayer& ly) {
      const Rsrc qr = rsrc(ly.W[0], (int64_t)a.H * D * dim), kr = rsrc(ly.W[1], (int64_t)a.Hkv * D * dim);
      const Rsrc vr = rsrc(ly.W[2], (int64_t)a.Hkv * D * dim);
      const int nq = h * D + 16 * w4 + col, nk = g * D + 16 * ds + col;
#pragma unroll
      for (int i = 0; i < VS; ++i) {
        const int s = w4 * VS + i;
        if (s < KST) {
          const uint32_t k = (uint32_t)(s * 64 + kg * 16);
          dma16(kr, blk + (KST + i) * 1024, (uint32_t)(nk * dim) + k);
          dma16(vr, blk + (KST + VS + i) * 1024, (uint32_t)(nk * dim) + k);
        }
      }
#pragma unroll
      for (int s = 0; s < KST; ++s) dma16(qr, blk + s * 1024, (uint32_t)(nq * dim + s * 64 + kg * 16));
    };
    // Attention layout: thread tid holds chunk kc = tid % 4 (16 key bytes, 4 value bytes of the
    // slice) of keys t = tid / 4 + 128 i, i < KR: the four threads of a key meet by DPP within a
    // quad, so scores, probabilities and products never leave the registers.
    const int kc = tid & 3, k0 = tid >> 2;
    v4i kreg[KR];
    int32_t vreg[KR];
    auto kv_issue = [&](const CLayer& ly) {  // the cache rows of earlier launches (positions < T - 1)
      const Rsrc krr = rsrc(ly.kc + (int64_t)g * a.max_seq * D, (int64_t)a.max_seq * D);
      const Rsrc vrr = rsrc(ly.vc + (int64_t)g * a.max_seq * D, (int64_t)a.max_seq * D);
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        const int t = k0 + 128 * i;
        kreg[i] = ld16(krr, t < T - 1 ? (uint32_t)(t * D + 16 * kc) : LD_OOB);
        vreg[i] = ld4(vrr, t < T - 1 ? (uint32_t)(t * D + 16 * ds + 4 * kc) : LD_OOB);
      }
    };
    if (alive) {
      if (!roww) w_issue(lyr[0]);
      kv_issue(lyr[0]);
    }
    for (int l = 0; l < a.L && alive; ++l) {
      const CLayer& ly = lyr[l];
      const int par = l & 1;
      const uint32_t ep = e0 + (uint32_t)l + 1u;
      v4i wop[PNL];
      if (roww) {
        RowOps fo;
        v2i rqc{0, 0};
        int32_t bc = 0;
        rowops_load(fo, l > 0 ? lyr[l - 1].rq_d : nullptr, l > 0 ? lyr[l - 1].bias_d : nullptr, ly.g1, dim, rt);
        if (wave < 3) {  // epilogue columns: wave 0 q (h D + lane), wave 1 k and wave 2 v (g D + 16 ds + lane)
          const int rl = wave;
          const int n = wave == 0 ? h * D + lane : g * D + 16 * ds + lane;
          const int nr = (rl == 0 ? a.H : a.Hkv) * D;
          const bool in = wave == 0 || lane < 16;
          rqc = ld8(rsrc(ly.rq[rl], (int64_t)nr * 8), in ? 8u * n : LD_OOB);
          bc = ld4(rsrc(ly.bias[rl], (int64_t)nr * 4), in ? 4u * n : LD_OOB);
        }
        const Rsrc pr = rsrc(ly.wo + (int64_t)h * dim * D, (int64_t)dim * D);
#pragma unroll
        for (int i = 0; i < PNL; ++i) {
          const int n = rt + 256 * i;
          wop[i] = ld16(pr, n < dim ? (uint32_t)(n * D + 16 * ds) : LD_OOB);
        }
        if (l > 0) {
          bool ok = true;
          if (wave == 0) ok = poll(a.fl3 + REP_WORDS * rep, a.nu3, ep - 1u, a.ctl, a.spin_max);
          if (!row_polled(ok)) {
            alive = false;
            break;
          }
        }
        int32_t x[4] = {0, 0, 0, 0};
        if (l > 0) {
          finish4(a.acc_d + (int64_t)(par ^ 1) * R * dim, a.xres + dim, fo, dim, rt, x);
        } else {
          const v2i xi = ld8(rsrc(a.x_in, (int64_t)dim * 2), 4 * rt < dim ? 8u * rt : LD_OOB);
          x[0] = lo16(xi.x);
          x[1] = hi16(xi.x);
          x[2] = lo16(xi.y);
          x[3] = hi16(xi.y);
        }
        if (u2 == 0 && 4 * rt < dim) {  // the layer input: the residual of this layer's S3
          v2i xo;
          xo.x = pack16(x[0], x[1]);
          xo.y = pack16(x[2], x[3]);
          stc8(rsrc(a.xres, (int64_t)dim * 2), 8u * rt, xo);
        }
        if (l == 0) {  // the launch's first accumulators start at zero (published below, fl0)
          const int n2 = 2 * R * dim, per = (n2 + a.nu2 - 1) / a.nu2;
          zero_slice(a, 0, u2 * per, std::min(n2, (u2 + 1) * per), rt);
        }
        if (!norm_quant(x, fo.g, (uint32_t)ly.eps1, (uint32_t)ly.C1, (int)ly.sh1, ly.Mq1, (int)ly.Sq1)) {
          alive = false;
          break;
        }
        sig_add(&sy.xrdy);
        if (wave == 1) {
          // the slice's k columns: requant16 + bias (golden.py:316-342) out as tagged words for the
          // head's four slices (RoPE and quant follow on the whole key, after the cached scores)
          nk += 4;
          if (!sig_wait(&sy.krdy, nk, &sy.abort)) {
            alive = false;
            break;
          }
          if (lane < 16) {
            const int32_t s = gk[0][lane] + gk[1][lane] + gk[2][lane] + gk[3][lane];
            const int32_t y = (int32_t)sat16(mulshift((int64_t)s + bc, (int64_t)rqc.x, rqc.y));
            stc4(rsrc(a.kx + (int64_t)h * D, 4 * D), 4u * (16 * ds + lane), ((ep & 0xFFFFu) << 16) | (uint32_t)(uint16_t)y);
          }
        } else if (wave != 3) {
          // q (wave 0): requant16 + bias, RoPE in 64-bit sums, quant (golden.py:316-342, 141-158,
          // 119-120); v slice (wave 2): requant8 + bias
          nw += 4;
          if (!sig_wait(&sy.wrdy, nw, &sy.abort)) {
            alive = false;
            break;
          }
          if (wave == 0) {
            const int32_t y = (int32_t)sat16(mulshift((int64_t)gq[lane] + bc, (int64_t)rqc.x, rqc.y));
            yq[lane] = y;
            if (lane < D / 2) {
              const int32_t x1 = yq[lane], x2 = yq[lane + D / 2];
              const int64_t r1 = (int64_t)x1 * cs - (int64_t)x2 * sn, r2 = (int64_t)x2 * cs + (int64_t)x1 * sn;
              const int32_t y1 = (int32_t)sat16(rshr(r1, 14)), y2 = (int32_t)sat16(rshr(r2, 14));
              const double sq = mulshift_scale(ly.quant_M[0], (int)ly.quant_S[0]);
              q8[lane] = (int8_t)mulshift_small_sat(y1, sq, -128.0, 127.0);
              q8[lane + D / 2] = (int8_t)mulshift_small_sat(y2, sq, -128.0, 127.0);
            }
          } else if (lane < 16) {
            const int32_t s = gv[0][lane] + gv[1][lane] + gv[2][lane] + gv[3][lane];
            const int8_t y = (int8_t)sat8(mulshift((int64_t)s + bc, (int64_t)rqc.x, rqc.y));
            vnew[lane] = y;
            if (kv_writer) ly.vc[((int64_t)g * a.max_seq + pos) * D + 16 * ds + lane] = y;  // the new value slice
          }
        }
        if (l == 0) {  // every unit's clearing stores done before any unit adds
          drain();
          if (!row_meet()) {
            alive = false;
            break;
          }
          if (wave == 0) publish(a.fl0, u2, a.nu2, ep);
        }
      } else {
        nx += 4;
        if (!sig_wait(&sy.xrdy, nx, &sy.abort)) {
          alive = false;
          break;
        }
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this layer's blocks (and cached keys)
        // first the slice's k columns (their exchange between the head's slices overlaps the rest):
        // K steps w VS .. w VS + VS - 1, every operand read at once (a step past the row meets a
        // zero block)
        {
          v4i ak = {0, 0, 0, 0}, xa[VS], bk[VS];
#pragma unroll
          for (int i = 0; i < VS; ++i) {
            xa[i] = *reinterpret_cast<const v4i*>(xq + min(w4 * VS + i, KST - 1) * 64 + kg * 16);
            bk[i] = lds16(blk + (KST + i) * 1024);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < VS; ++i) ak = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], bk[i], ak, 0, 0, 0);
          if (lane < 16) gk[w4][lane] = ak.x;  // one input row: every output row equals row 0
          sig_add(&sy.krdy);
        }
        // q tile w (all K steps) and the v columns' steps w VS ..: four K steps' operands read at
        // once, then their products (the LDS latency of a group is paid once)
        v4i aq = {0, 0, 0, 0}, av = {0, 0, 0, 0};
#pragma unroll
        for (int s0 = 0; s0 < KST; s0 += 4) {
          v4i xa[4], bq[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int s = min(s0 + u, KST - 1);
            xa[u] = *reinterpret_cast<const v4i*>(xq + s * 64 + kg * 16);
            bq[u] = lds16(blk + s * 1024);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (s0 + u < KST) aq = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[u], bq[u], aq, 0, 0, 0);
        }
        {
          v4i xa[VS], bv[VS];
#pragma unroll
          for (int i = 0; i < VS; ++i) {
            xa[i] = *reinterpret_cast<const v4i*>(xq + min(w4 * VS + i, KST - 1) * 64 + kg * 16);
            bv[i] = lds16(blk + (KST + VS + i) * 1024);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < VS; ++i) av = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], bv[i], av, 0, 0, 0);
        }
        if (lane < 16) {
          gq[16 * w4 + lane] = aq.x;
          gv[w4][lane] = av.x;
        }
        sig_add(&sy.wrdy);
        nw += 4;
      }
      // ---- attention over T keys on all eight waves (golden.py:162-180) ----
      if (!all_meet()) {  // q8 and vnew in LDS
        alive = false;
        break;
      }
      // the new key (position tn) belongs to the quad k0 = tn % 128, in wave kwave; that wave
      // requests the head's k words now and takes them after its cached keys' scores
      const int tn = T - 1;
      const bool kwave = wave == ((tn & 127) >> 4);
      const uint32_t kw0 = kwave ? ldc4(rsrc(a.kx + (int64_t)h * D, 4 * D), 4u * lane) : 0u;
      const v4i qv = *reinterpret_cast<const v4i*>(q8 + 16 * kc);
      const int32_t vnw = *reinterpret_cast<const int32_t*>(vnew + 4 * kc);
      int32_t sreg[KR];
      int32_t lmax = INT32_MIN;
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        const int t = k0 + 128 * i;
        sreg[i] = quad_sum(dot16(qv, kreg[i]));
        if (t < tn) lmax = max(lmax, sreg[i]);
      }
      if (KR * 128 < T) {  // keys past the registers (long contexts): scores into sc[]
        const Rsrc krr = rsrc(ly.kc + (int64_t)g * a.max_seq * D, (int64_t)a.max_seq * D);
        for (int tb0 = KR * 128; tb0 < T; tb0 += 4 * 128) {
          v4i kx[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int t = tb0 + 128 * u + k0;
            kx[u] = ld16(krr, t < T - 1 ? (uint32_t)(t * D + 16 * kc) : LD_OOB);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int t = tb0 + 128 * u + k0;
            const int32_t s = quad_sum(dot16(qv, kx[u]));
            if (t < tn) {
              if (kc == 0) sc[t] = s;
              lmax = max(lmax, s);
            }
          }
        }
      }
      if (kwave) {
        // the new key: the head's k from its four slices, RoPE in 64-bit sums and quant
        // (golden.py:141-158, 119-120), its cache row (golden.py:344-351), its score
        int32_t y = 0;
        if (!take_tagged(a.kx + (int64_t)h * D, ep & 0xFFFFu, kw0, a.ctl, a.spin_max, y)) {
          alive = false;
          break;
        }
        yk[lane] = y;
        if (lane < D / 2) {
          const int32_t x1 = yk[lane], x2 = yk[lane + D / 2];
          const int64_t r1 = (int64_t)x1 * cs - (int64_t)x2 * sn, r2 = (int64_t)x2 * cs + (int64_t)x1 * sn;
          const int32_t y1 = (int32_t)sat16(rshr(r1, 14)), y2 = (int32_t)sat16(rshr(r2, 14));
          const double sq = mulshift_scale(ly.quant_M[1], (int)ly.quant_S[1]);
          const int8_t q1 = (int8_t)mulshift_small_sat(y1, sq, -128.0, 127.0);
          const int8_t q2 = (int8_t)mulshift_small_sat(y2, sq, -128.0, 127.0);
          k8[lane] = q1;
          k8[lane + D / 2] = q2;
          if (kv_writer && ds == 0) {
            const int64_t krow = ((int64_t)g * a.max_seq + pos) * D;
            ly.kc[krow + lane] = q1;
            ly.kc[krow + lane + D / 2] = q2;
          }
        }
        if (k0 == (tn & 127)) {
          const int32_t s = quad_sum(dot16(qv, *reinterpret_cast<const v4i*>(k8 + 16 * kc)));
          lmax = max(lmax, s);
          if (tn >= KR * 128) {
            if (kc == 0) sc[tn] = s;
          } else {
#pragma unroll
            for (int i = 0; i < KR; ++i)
              if (i == (tn >> 7)) sreg[i] = s;
          }
        }
      }
      lmax = wave_max_i32(lmax);
      if (lane == 0) redmax[wave] = lmax;
      if (!all_meet()) {
        alive = false;
        break;
      }
      int32_t mx = redmax[0];
#pragma unroll
      for (int w = 1; w < 8; ++w) mx = max(mx, redmax[w]);
      // probabilities (golden.py:168-172); each key's four threads compute it, its first adds it
      uint32_t pv[KR];
      uint32_t lsum = 0;
      const uint32_t Ms = (uint32_t)ly.Ms;
      const int Ss = (int)ly.Ss;
      const uint64_t zhalf = Ss > 0 ? 1ull << (Ss - 1) : 0ull;
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        const int t = k0 + 128 * i;
        pv[i] = t < T ? prob_gap(mx - sreg[i], Ms, zhalf, Ss, ei, ef) : 0u;
        if (kc == 0) lsum += pv[i];
      }
      if (KR * 128 < T) {
        for (int t = KR * 128 + k0; t < T; t += 128) {
          const uint32_t p = prob_gap(mx - sc[t], Ms, zhalf, Ss, ei, ef);
          if (kc == 0) lsum += p;
        }
      }
      lsum = (uint32_t)wave_sum_i32((int)lsum);  // T * 65535 < 2^31
      if (lane == 0) redsum[wave] = (int32_t)lsum;
      if (!all_meet()) {
        alive = false;
        break;
      }
      uint32_t total = 0;
#pragma unroll
      for (int w = 0; w < 8; ++w) total += (uint32_t)redsum[w];
      const uint32_t inv = 0x80000000u / (total > 1u ? total : 1u);  // udiv(2^31, total), golden.py:174
      const int pb = (int)ly.pb, shp = 31 - pb;
      const int32_t cap = (1 << pb) - 1;
      const uint64_t phalf = 1ull << (shp - 1);
      // o[j] = sum_t pn[t] * v[t][16 ds + 4 kc + j]
      int32_t o[4] = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        const int t = k0 + 128 * i;
        const int32_t pn = prob_norm(pv[i], inv, phalf, shp, cap);
        const int32_t vw = t == T - 1 ? vnw : vreg[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] += pn * sbyte(vw, j);
      }
      if (KR * 128 < T) {  // keys past the registers
        const Rsrc vrr = rsrc(ly.vc + (int64_t)g * a.max_seq * D, (int64_t)a.max_seq * D);
        for (int t = KR * 128 + k0; t < T; t += 128) {
          const uint32_t p = prob_gap(mx - sc[t], Ms, zhalf, Ss, ei, ef);
          const int32_t pn = prob_norm(p, inv, phalf, shp, cap);
          const int32_t vw = t == T - 1 ? vnw : ld4(vrr, (uint32_t)(t * D + 16 * ds + 4 * kc));
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] += pn * sbyte(vw, j);
        }
      }
      // the 16 lanes of a row with equal lane % 4 hold the same four dimensions: fold them, then the
      // 4 rows x 8 waves partials in LDS
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[j] += dpp_mov<DPP_ROW_ROR + 4>(o[j]);
        o[j] += dpp_mov<DPP_ROW_ROR + 8>(o[j]);
      }
      if ((lane & 15) < 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) wpart[4 * wave + (lane >> 4)][4 * kc + j] = o[j];
      }
      if (!all_meet()) {
        alive = false;
        break;
      }
      if (!roww) {
        // the next layer's blocks and cached keys/values, requested once the row waves' atomics
        // have landed and the flag is on its way (ahead of these loads in the CU's memory queue;
        // the row waves request their keys after the flag)
        if (l + 1 < a.L) {
          __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (!sig_wait(&sy.aiss, 4u * (uint32_t)(l + 1), &sy.abort)) {
            alive = false;
            break;
          }
          w_issue(lyr[l + 1]);
          kv_issue(lyr[l + 1]);
        }
        continue;
      }
      if (wave == 0 && lane < 16) {
        int32_t s = 0;
#pragma unroll
        for (int r = 0; r < 32; ++r) s += wpart[r][lane];
        if (ly.pb == 15) s = rshr32(s, 7);  // golden.py:177-178
        ah[lane] = (int8_t)sat8(mulshift(s, ly.Mo, (int)ly.So));
      }
      if (l == 0) {  // every unit's clearing done (the row waves' wait on fl0)
        bool ok = true;
        if (wave == 0) ok = poll(a.fl0 + REP_WORDS * rep, a.nu2, ep, a.ctl, a.spin_max);
        if (!row_polled(ok)) {
          alive = false;
          break;
        }
      } else if (!row_meet()) {
        alive = false;
        break;
      }
      // the slice's output-projection partial sums (golden.py:316-342, K range h D + 16 ds ..)
      const v4i avv = *reinterpret_cast<const v4i*>(ah);
      int32_t* acc = a.acc_o + ((int64_t)par * R + (u2 % R)) * dim;
#pragma unroll
      for (int i = 0; i < PNL; ++i) {
        const int n = rt + 256 * i;
        const int32_t s = dot16(avv, wop[i]);
        if (n < dim && s != 0) atomic_add_dev(acc + n, s);
      }
      drain();
      if (!row_meet()) {
        alive = false;
        break;
      }
      if (wave == 0) publish(a.fl2, u2, a.nu2, ep);
      sig_add(&sy.aiss);
      if (l + 1 < a.L) kv_issue(lyr[l + 1]);
    }
  } else if (u3 >= 0) {
    // =============================== S3 unit (tiles ta, tb) ===============================
    // weight wave w: gate (w < 2) or up, K half w & 1: blocks [0, NS3) tile ta, [NS3, 2 NS3) tile tb
    auto w_issue = [&](const CLayer& ly) {
      const int mat = w4 >> 1, kh = w4 & 1, s0 = kh * NS3;
      const Rsrc wr = rsrc(mat ? ly.Wu : ly.Wg, (int64_t)a.F * dim);
      const int na = 16 * ta + col, nb = 16 * tb + col;
#pragma unroll
      for (int u = 0; u < NS3; ++u) {
        const int s = s0 + u;
        const uint32_t k = (uint32_t)(s * 64 + kg * 16);
        if (s < KST) {  // blocks past the row, and those of an absent tile, are never loaded: zero
          dma16(wr, blk + u * 1024, (uint32_t)(na * dim) + k);
          if (tb >= 0) dma16(wr, blk + (NS3 + u) * 1024, (uint32_t)(nb * dim) + k);
        }
      }
    };
    if (alive && !roww) w_issue(lyr[0]);
    for (int l = 0; l < a.L && alive; ++l) {
      const CLayer& ly = lyr[l];
      const int par = l & 1;
      const uint32_t ep = e0 + (uint32_t)l + 1u;
      if (roww) {
        RowOps fo;
        v2i rqg{0, 0}, rqu{0, 0};
        int32_t bgv = 0, buv = 0;
        v4i wda[PNL], wdb[PNL];
        // wave 0's epilogue lanes: kg 0 = tile ta's column col, kg 1 = tile tb's
        const int en = kg == 0 ? 16 * ta + col : (kg == 1 && tb >= 0 ? 16 * tb + col : a.F);
        rowops_load(fo, ly.rq_o, ly.bias_o, ly.g2, dim, rt);
        if (wave == 0) {
          const bool mine = en < a.F;
          const uint32_t o8 = mine ? 8u * en : LD_OOB, o4 = mine ? 4u * en : LD_OOB;
          rqg = ld8(rsrc(ly.rqg, (int64_t)a.F * 8), o8);
          rqu = ld8(rsrc(ly.rqu, (int64_t)a.F * 8), o8);
          bgv = ld4(rsrc(ly.bg, (int64_t)a.F * 4), o4);
          buv = ld4(rsrc(ly.bu, (int64_t)a.F * 4), o4);
        }
        const Rsrc dr = rsrc(ly.wd, (int64_t)a.tiles * dim * 16);
#pragma unroll
        for (int i = 0; i < PNL; ++i) {
          const int n = rt + 256 * i;
          const bool in = n < dim;
          wda[i] = ld16(dr, in ? (uint32_t)(((int64_t)ta * dim + n) * 16) : LD_OOB);
          wdb[i] = ld16(dr, (in && tb >= 0) ? (uint32_t)(((int64_t)tb * dim + n) * 16) : LD_OOB);
        }
        bool ok = true;
        if (wave == 0) ok = poll(a.fl2 + REP_WORDS * rep, a.nu2, ep, a.ctl, a.spin_max);
        if (!row_polled(ok)) {
          alive = false;
          break;
        }
        int32_t x[4] = {0, 0, 0, 0};
        finish4(a.acc_o + (int64_t)par * R * dim, a.xres, fo, dim, rt, x);
        if (u3 == 0 && 4 * rt < dim) {  // the attention residual x1: the next layer's S12 adds to it
          v2i xo;
          xo.x = pack16(x[0], x[1]);
          xo.y = pack16(x[2], x[3]);
          stc8(rsrc(a.xres + dim, (int64_t)dim * 2), 8u * rt, xo);
        }
        // the next layer's accumulators (parity par ^ 1): their last readers are done
        const int n2 = 2 * R * dim, per = (n2 + a.nu3 - 1) / a.nu3;
        zero_slice(a, par ^ 1, u3 * per, std::min(n2, (u3 + 1) * per), rt);
        if (!norm_quant(x, fo.g, (uint32_t)ly.eps2, (uint32_t)ly.C2, (int)ly.sh2, ly.Mq2, (int)ly.Sq2)) {
          alive = false;
          break;
        }
        sig_add(&sy.xrdy);
        if (wave == 0) {
          nw += 4;
          if (!sig_wait(&sy.wrdy, nw, &sy.abort)) {
            alive = false;
            break;
          }
          if (kg < 2) {
            // gate (SiLU) and up (mul) epilogues, quant (golden.py:316-342, 101-107, 119-120) in the
            // exact 32-bit / double forms of the decode chain (|tg|, |tu| < 2^15, |tu * sg| < 2^31)
            const int tl = kg;
            int8_t fq = 0;
            if (en < a.F) {
              const int32_t ag = red3[tl][0][col] + red3[tl][1][col], au = red3[tl][2][col] + red3[tl][3][col];
              const int64_t tg = sat16(mulshift((int64_t)ag + bgv, rqg.x, rqg.y));
              const int64_t tu = sat16(mulshift((int64_t)au + buv, rqu.x, rqu.y));
              const int32_t sg =
                  silu16_fast((int32_t)tg, mulshift_scale(ly.silu_Mi, (int)ly.silu_Si), (int)ly.silu_sh, sig);
              const int32_t f = min(max(rshr32_any((int32_t)tu * sg, (int)ly.mul_sh), -32768), 32767);
              fq = (int8_t)mulshift_small_sat(f, mulshift_scale(ly.fq_M, (int)ly.fq_S), -128.0, 127.0);
            }
            fq16[tl][col] = fq;
          }
        }
        if (!row_meet()) {
          alive = false;
          break;
        }
        const v4i fa = *reinterpret_cast<const v4i*>(fq16[0]);
        const v4i fb = *reinterpret_cast<const v4i*>(fq16[1]);
        int32_t* acc = a.acc_d + ((int64_t)par * R + (u3 % R)) * dim;
#pragma unroll
        for (int i = 0; i < PNL; ++i) {
          const int n = rt + 256 * i;
          const int32_t d = dot16(fb, wdb[i], dot16(fa, wda[i]));
          if (n < dim && d != 0) atomic_add_dev(acc + n, d);
        }
        drain();
        if (!row_meet()) {
          alive = false;
          break;
        }
        if (wave == 0) publish(a.fl3, u3, a.nu3, ep);
        sig_add(&sy.aiss);
      } else {
        nx += 4;
        if (!sig_wait(&sy.xrdy, nx, &sy.abort)) {
          alive = false;
          break;
        }
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this layer's blocks
        const int kh = w4 & 1, s0 = kh * NS3;
        v4i am = {0, 0, 0, 0}, at = {0, 0, 0, 0};
#pragma unroll
        for (int u0 = 0; u0 < NS3; u0 += 4) {  // four steps' operands read at once
          v4i xa[4], ba[4], bb[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int uu = min(u0 + u, NS3 - 1);
            const int s = min(s0 + uu, KST - 1);  // (a step past the row meets zero blocks)
            xa[u] = *reinterpret_cast<const v4i*>(xq + s * 64 + kg * 16);
            ba[u] = lds16(blk + uu * 1024);
            bb[u] = lds16(blk + (NS3 + uu) * 1024);
          }
          __builtin_amdgcn_sched_barrier(0);  // all twelve reads issued before the first product
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (u0 + u < NS3) {
              am = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[u], ba[u], am, 0, 0, 0);
              at = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[u], bb[u], at, 0, 0, 0);
            }
          }
        }
        if (lane < 16) {
          red3[0][w4][lane] = am.x;
          red3[1][w4][lane] = at.x;
        }
        sig_add(&sy.wrdy);
        nw += 4;
        // the next layer's blocks, requested once this wave's reads are done and the row waves'
        // atomics have landed and the flag is on its way (ahead of these loads in the CU's queue)
        if (l + 1 < a.L) {
          __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (!sig_wait(&sy.aiss, 4u * (uint32_t)(l + 1), &sy.abort)) {
            alive = false;
            break;
          }
          w_issue(lyr[l + 1]);
        }
      }
    }
  }
  // a wave that left the loop early tells the others (their waits end)
  if (!alive) __hip_atomic_store(&sy.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into this workgroup's LDS outlives it
  __syncthreads();
  // launch count: the last workgroup to finish advances it (the next launch's epochs)
  if (tid == 0) {
    const uint32_t done = __hip_atomic_fetch_add(a.ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == (uint32_t)G - 1u) {
      __hip_atomic_store(a.ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctl + 0, seq + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace dstep
}  // namespace llhip

using namespace llhip;
using namespace llhip::dstep;

struct llhip_dec_step {
  Args a{};
  int kst = 0, G = 0;
  size_t lds = 0;
  void* mem = nullptr;  // layer table + state, one allocation
};

namespace {

template <int KST>
size_t step_lds(int max_seq) {
  return (size_t)StepCfg<KST>::SC_OFF + (size_t)max_seq * 4;
}

template <int KST>
int launch_step(const llhip_dec_step* s, void* stream) {
  const size_t lds = step_lds<KST>(s->a.max_seq);
  hipLaunchKernelGGL((dec_step_kernel<KST>), dim3(s->G), dim3(NTH), lds, (hipStream_t)stream, s->a);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

bool norm_ok(int64_t eps, int64_t C, int64_t sh, int64_t Mq, int64_t Sq) {
  return u32_ok(eps) && u32_ok(C) && shift_ok(sh) && u32_ok(Mq) && shift_ok(Sq);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" llhip_dec_step* llhip_dec_step_create(const llhip_dec_step_desc* d) {
  if (!d || !d->layers || d->L < 1 || d->L > 63) {
    fail(-EINVAL, "dec_step: 1..63 layers");
    return nullptr;
  }
  const int64_t dim = d->dim, H = d->H, Hkv = d->Hkv, F = d->F, S = d->max_seq;
  if (d->D != D) {
    fail(-EINVAL, "dec_step: head_dim %d only", D);
    return nullptr;
  }
  if (dim < 64 || dim % 64 || dim > MAX_DIM || H < 1 || Hkv < 1 || H % Hkv || F < 16 || F % 16 || S < 1 ||
      S > 8192 || F * dim >= (1ll << 31) || S * Hkv * D >= (1ll << 31) || H * D * dim >= (1ll << 31)) {
    fail(-EINVAL, "dec_step: unsupported geometry");
    return nullptr;
  }
  if (!d->x_in || !d->cos_tab || !d->sin_tab || !d->pos_dev) {
    fail(-EINVAL, "dec_step: null operand");
    return nullptr;
  }
  const int G = std::min(current_cu_count(), MAX_G);
  const int64_t nu2 = H * (D / 16), tiles = F / 16;
  const int64_t w3 = G - nu2;  // workgroups left for S3, each taking tiles u and u + w3
  if (nu2 > 256 || w3 < 1 || tiles > 2 * w3) {
    fail(-EINVAL, "dec_step: %lld attention units and %lld FFN tiles do not fit %d workgroups", (long long)nu2,
         (long long)tiles, G);
    return nullptr;
  }
  const int64_t nu3 = std::min(w3, tiles);
  std::vector<Layer> tab((size_t)d->L);
  for (int64_t l = 0; l < d->L; ++l) {
    const llhip_step_layer& s = d->layers[l];
    Layer& t = tab[(size_t)l];
    if (!s.g1 || !s.g2 || !s.kc || !s.vc || !s.wo_panel || !s.rq_o || !s.Wg || !s.Wu || !s.rqg || !s.rqu ||
        !s.wd_panel || !s.rq_d) {
      fail(-EINVAL, "dec_step: layer %lld has a null operand", (long long)l);
      return nullptr;
    }
    for (int i = 0; i < 3; ++i)
      if (!s.W[i] || !s.rq[i]) {
        fail(-EINVAL, "dec_step: layer %lld q/k/v operands", (long long)l);
        return nullptr;
      }
    if (!norm_ok(s.eps1, s.C1, s.sh1, s.Mq1, s.Sq1) || !norm_ok(s.eps2, s.C2, s.sh2, s.Mq2, s.Sq2) ||
        !u32_ok(s.quant_M[0]) || !u32_ok(s.quant_M[1]) || !shift_ok(s.quant_S[0]) || !shift_ok(s.quant_S[1]) ||
        !shift_ok(s.Ss) || !shift_ok(s.So) || !u32_ok(s.Ms) || !(s.prob_bits == 8 || s.prob_bits == 15) || !u32_ok(s.silu_Mi) ||
        !shift_ok(s.silu_Si) || !shift_ok(s.silu_sh) || !shift_ok(s.mul_sh) || !u32_ok(s.fq_M) || !shift_ok(s.fq_S)) {
      fail(-EINVAL, "dec_step: layer %lld parameter out of range", (long long)l);
      return nullptr;
    }
    if (!al16(s.g1) || !al16(s.g2) || !al16(s.rq_o) || !al16(s.rq_d) || (s.bias_o && !al16(s.bias_o)) ||
        (s.bias_d && !al16(s.bias_d)) || !al16(s.wo_panel) || !al16(s.wd_panel) || !al16(s.W[0]) ||
        !al16(s.W[1]) || !al16(s.W[2]) || !al16(s.Wg) || !al16(s.Wu)) {
      fail(-EINVAL, "dec_step: layer %lld operands must be 16-byte aligned", (long long)l);
      return nullptr;
    }
    t.g1 = static_cast<const int16_t*>(s.g1);
    for (int i = 0; i < 3; ++i) {
      t.W[i] = static_cast<const int8_t*>(s.W[i]);
      t.rq[i] = static_cast<const int32_t*>(s.rq[i]);
      t.bias[i] = static_cast<const int32_t*>(s.bias[i]);
    }
    t.kc = static_cast<int8_t*>(s.kc);
    t.vc = static_cast<int8_t*>(s.vc);
    t.wo = static_cast<const int8_t*>(s.wo_panel);
    t.rq_o = static_cast<const int32_t*>(s.rq_o);
    t.bias_o = static_cast<const int32_t*>(s.bias_o);
    t.g2 = static_cast<const int16_t*>(s.g2);
    t.Wg = static_cast<const int8_t*>(s.Wg);
    t.Wu = static_cast<const int8_t*>(s.Wu);
    t.rqg = static_cast<const int32_t*>(s.rqg);
    t.rqu = static_cast<const int32_t*>(s.rqu);
    t.bg = static_cast<const int32_t*>(s.bg);
    t.bu = static_cast<const int32_t*>(s.bu);
    t.wd = static_cast<const int8_t*>(s.wd_panel);
    t.rq_d = static_cast<const int32_t*>(s.rq_d);
    t.bias_d = static_cast<const int32_t*>(s.bias_d);
    t.Mq1 = s.Mq1;
    t.Mq2 = s.Mq2;
    t.quant_M[0] = s.quant_M[0];
    t.quant_M[1] = s.quant_M[1];
    t.Ms = s.Ms;
    t.Mo = s.Mo;
    t.silu_Mi = s.silu_Mi;
    t.fq_M = s.fq_M;
    t.eps1 = s.eps1;
    t.C1 = s.C1;
    t.eps2 = s.eps2;
    t.C2 = s.C2;
    t.sh1 = s.sh1;
    t.Sq1 = s.Sq1;
    t.sh2 = s.sh2;
    t.Sq2 = s.Sq2;
    t.quant_S[0] = s.quant_S[0];
    t.quant_S[1] = s.quant_S[1];
    t.Ss = s.Ss;
    t.So = s.So;
    t.pb = s.prob_bits;
    t.silu_Si = s.silu_Si;
    t.silu_sh = s.silu_sh;
    t.mul_sh = s.mul_sh;
    t.fq_S = s.fq_S;
  }
  const int kst = (int)(dim / 64);  // K steps of 64: the kernel is compiled for 9, 14 and 16
  if (kst != 9 && kst != 14 && kst != 16) {
    fail(-EINVAL, "dec_step: dim %lld is not one of 576, 896, 1024", (long long)dim);
    return nullptr;
  }
  const size_t lds = kst == 9 ? step_lds<9>((int)S) : kst == 14 ? step_lds<14>((int)S) : step_lds<16>((int)S);
  if (lds > 150 * 1024) {  // 160 KiB per CU, of which the kernel's fixed arrays take a few
    fail(-EINVAL, "dec_step: %zu bytes of LDS (dim %lld, max_seq %lld) exceed the CU", lds, (long long)dim,
         (long long)S);
    return nullptr;
  }
  // Workgroup roles.  Workgroup b runs on XCD b % 8 (dispatch is round-robin over the XCDs), so
  // the DC slices of head h go to workgroups b = 8 (DC (h / 8) + ds) + h % 8: one XCD, whose L2
  // then serves the head's q rows once for its slices.  The S3 units take the rest in order.
  std::vector<int32_t> role((size_t)G, -1);
  {
    bool xcd = G % 8 == 0;
    for (int64_t u = 0; u < nu2 && xcd; ++u) xcd = 8 * (DC * (u / DC / 8) + u % DC) + (u / DC) % 8 < G;
    for (int64_t u = 0; u < nu2; ++u) {
      const int64_t h = u / DC, b = xcd ? 8 * (DC * (h / 8) + u % DC) + h % 8 : u;
      role[(size_t)b] = (int32_t)u;
    }
    int64_t u3 = 0;
    for (int64_t b = 0; b < G && u3 < nu3; ++b)
      if (role[(size_t)b] < 0) role[(size_t)b] = (int32_t)(256 + u3++);
  }
  // one allocation: layer table | ctl (256 B) | roles (1 KiB) | flags 3 x NREP x 4 KiB | k exchange |
  // acc_o | acc_d | xres
  const size_t tab_b = (sizeof(Layer) * (size_t)d->L + 255) & ~(size_t)255;
  const size_t acc_b = (size_t)2 * R * dim * 4;
  const size_t off_ctl = tab_b, off_role = off_ctl + 256, off_fl = off_role + 4 * MAX_G,
               off_kx = off_fl + 3 * FLAG_WORDS * 4, off_ao = off_kx + (((size_t)H * D * 4 + 255) & ~(size_t)255),
               off_ad = off_ao + acc_b, off_x = off_ad + acc_b,
               total = off_x + ((size_t)(2 * dim * 2 + 255) & ~(size_t)255);
  llhip_dec_step* s = new llhip_dec_step();
  if (hipMalloc(&s->mem, total) != hipSuccess) {
    fail(-EIO, "dec_step: device allocation failed");
    delete s;
    return nullptr;
  }
  char* m = static_cast<char*>(s->mem);
  if (hipMemset(m, 0, total) != hipSuccess ||
      hipMemcpy(m, tab.data(), sizeof(Layer) * (size_t)d->L, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(m + off_role, role.data(), 4 * (size_t)G, hipMemcpyHostToDevice) != hipSuccess) {
    fail(-EIO, "dec_step: upload failed");
    (void)hipFree(s->mem);
    delete s;
    return nullptr;
  }
  Args& a = s->a;
  a.layers = reinterpret_cast<const Layer*>(m);
  a.x_in = static_cast<const int16_t*>(d->x_in);
  a.cos_tab = static_cast<const int16_t*>(d->cos_tab);
  a.sin_tab = static_cast<const int16_t*>(d->sin_tab);
  a.pos_dev = static_cast<const int32_t*>(d->pos_dev);
  a.ctl = reinterpret_cast<uint32_t*>(m + off_ctl);
  a.role = reinterpret_cast<const int32_t*>(m + off_role);
  a.fl0 = reinterpret_cast<uint32_t*>(m + off_fl);
  a.fl2 = reinterpret_cast<uint32_t*>(m + off_fl + FLAG_WORDS * 4);
  a.fl3 = reinterpret_cast<uint32_t*>(m + off_fl + 2 * FLAG_WORDS * 4);
  a.kx = reinterpret_cast<uint32_t*>(m + off_kx);
  a.acc_o = reinterpret_cast<int32_t*>(m + off_ao);
  a.acc_d = reinterpret_cast<int32_t*>(m + off_ad);
  a.xres = reinterpret_cast<int16_t*>(m + off_x);
  a.L = (int)d->L;
  a.dim = (int)dim;
  a.H = (int)H;
  a.Hkv = (int)Hkv;
  a.max_seq = (int)S;
  a.F = (int)F;
  a.nu2 = (int)nu2;
  a.nu3 = (int)nu3;
  a.tiles = (int)tiles;
  a.spin_max = 1u << 20;
  s->kst = kst;
  s->G = G;
  s->lds = lds;
  return s;
}

extern "C" int llhip_dec_step_run(llhip_dec_step* s, void* stream) {
  if (!s) return fail(-EINVAL, "dec_step: null step");
  if (s->kst == 9) return launch_step<9>(s, stream);
  if (s->kst == 14) return launch_step<14>(s, stream);
  return launch_step<16>(s, stream);
}

extern "C" int llhip_dec_step_outputs(llhip_dec_step* s, void** acc, void** resid) {
  if (!s || !acc || !resid) return fail(-EINVAL, "dec_step: null argument");
  const int par = (s->a.L - 1) & 1;
  *acc = s->a.acc_d + (int64_t)par * R * s->a.dim;
  *resid = s->a.xres + s->a.dim;
  return 0;
}

extern "C" int llhip_dec_step_status(llhip_dec_step* s, int64_t* launches, int64_t* err) {
  if (!s) return fail(-EINVAL, "dec_step: null step");
  uint32_t h[4];
  LLHIP_CHECK_HIP(hipDeviceSynchronize());
  LLHIP_CHECK_HIP(hipMemcpy(h, s->a.ctl, sizeof(h), hipMemcpyDeviceToHost));
  if (launches) *launches = h[0];
  if (err) *err = h[2];
  return 0;
}

extern "C" void llhip_dec_step_destroy(llhip_dec_step* s) {
  if (!s) return;
  if (s->mem) (void)hipFree(s->mem);
  delete s;
}
