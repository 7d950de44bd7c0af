// Shared device numerics and host plumbing of libllhip (gfx950).
//
// The device functions restate the integer contract of the reference's
// docs/NUMERICS.md ("Primitives") exactly as python/llaccel/golden.py computes
// it: every intermediate is an int64 and every product wraps modulo 2^64 (the
// reference's int64 numpy arithmetic), so results are bit-identical for every
// input the host side accepts.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cerrno>
#include <cstdio>
#include <string>

namespace llhip {

// ---------------------------------------------------------------------------------------
// error reporting (thread-local message, negative errno return codes)
// ---------------------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define LLHIP_CHECK_HIP(expr)                                                                   \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess) return ::llhip::fail(-EIO, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define LLHIP_LAUNCH_CHECK()                                                                       \
  do {                                                                                            \
    hipError_t e_ = hipGetLastError();                                                            \
    if (e_ != hipSuccess) return ::llhip::fail(-EIO, "kernel launch: %s", hipGetErrorString(e_)); \
  } while (0)

inline bool shift_ok(int64_t s) { return s >= 0 && s <= 63; }
inline bool u32_ok(int64_t v) { return v >= 0 && v <= 0xFFFFFFFFll; }

// ---------------------------------------------------------------------------------------
// device numerics (golden.py:35-120)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int64_t wmul(int64_t a, int64_t b) {
  return (int64_t)((uint64_t)a * (uint64_t)b);
}
// round-half-up arithmetic right shift, s in [0, 63] (golden.py:35-45)
__device__ __forceinline__ int64_t rshr(int64_t v, int s) {
  return s == 0 ? v : (v >> s) + ((v >> (s - 1)) & 1);
}
__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}
__device__ __forceinline__ int64_t sat8(int64_t v) { return clamp64(v, -128, 127); }
__device__ __forceinline__ int64_t sat16(int64_t v) { return clamp64(v, -32768, 32767); }
// golden.py:64-65
__device__ __forceinline__ int64_t mulshift(int64_t v, int64_t M, int s) { return rshr(wmul(v, M), s); }

// 32-bit fast path of rshr for values known to fit i32 after the shift's rounding
__device__ __forceinline__ int32_t rshr32(int32_t v, int s) {
  return s == 0 ? v : (v >> s) + ((v >> (s - 1)) & 1);
}

// rshr of an int32 by any shift in [0, 63]: for s >= 32, |v| <= 2^31 gives v / 2^s in [-1/2, 1/2)
// and the rounded result 0
__device__ __forceinline__ int32_t rshr32_any(int32_t v, int s) {
  return s == 0 ? v : (s >= 32 ? 0 : (v >> s) + ((v >> (s - 1)) & 1));
}

// mulshift(x, M, S) = floor(x * M / 2^S + 1/2) (golden.py:35-45, 64-65) for |x| <= 2^20, M < 2^32 and
// S in [0, 63], in double precision with `scale` = M * 2^-S (exact: M has 32 significant bits): x *
// scale + 1/2 is a multiple of 2^-(S+1) below 2^52 in magnitude, exact in the 53-bit significand for
// S <= 52, so the fused multiply-add rounds nothing; for S > 52 |x * scale| < 2^-1 and the rounded sum
// stays inside (0, 1), whose floor 0 is the exact one.  Four full-rate instructions instead of 64-bit
// multiplies.
__device__ __forceinline__ double mulshift_scale(int64_t M, int S) { return __builtin_ldexp((double)M, -S); }
__device__ __forceinline__ int32_t mulshift_small_sat(int32_t x, double scale, double lo, double hi) {
  const double v = __builtin_floor(__builtin_fma((double)x, scale, 0.5));
  return (int32_t)__builtin_fmin(__builtin_fmax(v, lo), hi);
}

// silu16 (golden.py:101-107) of an i16-range x with the SIG table in LDS, exactly, in 32-bit and
// double arithmetic: u = sat16(mulshift(x, Mi, Si)) by mulshift_small_sat; SIG values are below
// 2^16, so x * sg lies in [-2^31, 2^31) and its rounding shift is rshr32_any.
__device__ __forceinline__ int32_t silu16_fast(int32_t x, double smul, int sh, const uint16_t* sig) {
  const int32_t u = mulshift_small_sat(x, smul, -32768.0, 32767.0);
  const int j = (u >> 8) + 128;
  const int32_t f = u & 255;
  const int32_t lo = sig[j], hi = sig[j + 1];
  const int32_t sg = lo + (((hi - lo) * f) >> 8);
  return min(max(rshr32_any(x * sg, sh), -32768), 32767);
}

// floor(sqrt(t)) for t < 2^48 (golden.py:68-81 computes it by the restoring method, two bits
// per step).  t converts to double exactly and its square root is within a few ulp (< 2^-26
// here) of sqrt(t), so the truncated root r is floor(sqrt(t)) or, when t = n^2 and the rounded
// root lands just below n, n - 1; one exact integer check (r + 1)^2 <= t repairs that case.
__device__ __forceinline__ uint32_t isqrt48(uint64_t t) {
  uint32_t r = (uint32_t)__builtin_sqrt((double)t);
  const uint64_t r1 = (uint64_t)r + 1;
  if (r1 * r1 <= t) r = (uint32_t)r1;
  else if ((uint64_t)r * r > t) --r;
  return r;
}

// LUTs generated by llaccel_amd/luts.py (luts.py:18-29 of the reference); one
// __constant__ copy per translation unit (no relocatable device code)
#include "luts.inc"

// golden.py:101-107
__device__ __forceinline__ int64_t silu16(int64_t x, int64_t Mi, int Si, int sh) {
  int64_t u = sat16(mulshift(x, Mi, Si));
  int j = (int)((u >> 8) + 128);
  int64_t f = u & 255;
  int64_t lo = kSig[j], hi = kSig[j + 1];
  int64_t sg = lo + (((hi - lo) * f) >> 8);
  return sat16(rshr(wmul(x, sg), sh));
}

// silu16 with the SIG table staged in LDS (kSig copied by the kernel)
__device__ __forceinline__ int64_t silu16_lds(int64_t x, int64_t Mi, int Si, int sh, const uint16_t* sig) {
  int64_t u = sat16(mulshift(x, Mi, Si));
  int j = (int)((u >> 8) + 128);
  int64_t f = u & 255;
  int64_t lo = sig[j], hi = sig[j + 1];
  int64_t sg = lo + (((hi - lo) * f) >> 8);
  return sat16(rshr(wmul(x, sg), sh));
}

// silu16_lds for |x| < 2^15 and 0 <= Mi < 2^32 (every i16 GEMM output; the host checks Mi is u32):
// x * Mi is one signed x unsigned 32 x 32 -> 64 product (|x * Mi| < 2^47), rshr(v, S) is
// (v + 2^(S-1)) >> S, and x * sg (|sg| < 2^16) fits 32 bits
__device__ __forceinline__ int32_t silu16_i16(int32_t x, uint32_t Mi, int Si, int sh, const uint16_t* sig) {
  const int64_t prod = (int64_t)x * (int64_t)Mi;
  const int64_t v = Si > 0 ? (prod + ((int64_t)1 << (Si - 1))) >> Si : prod;
  const int32_t u = (int32_t)clamp64(v, -32768, 32767);
  const int j = (u >> 8) + 128;
  const int32_t f = u & 255;
  const int32_t lo = sig[j], hi = sig[j + 1];
  const int32_t sg = lo + (((hi - lo) * f) >> 8);
  const int64_t w = (int64_t)(x * sg);
  const int64_t y = sh > 0 ? (w + ((int64_t)1 << (sh - 1))) >> sh : w;
  return (int32_t)clamp64(y, -32768, 32767);
}

// exp LUT probability of a nonnegative scaled score gap (golden.py:170-172)
__device__ __forceinline__ uint32_t lut_prob(int64_t z) {
  if (z >= 4096 || z < 0) return 0u;
  uint32_t zi = (uint32_t)z;
  return ((uint32_t)kExpI[zi >> 8] * (uint32_t)kExpF[zi & 255] + 32768u) >> 16;
}

// ---------------------------------------------------------------------------------------
// shared vector helpers
// ---------------------------------------------------------------------------------------
// Wave reductions on the DPP datapath: quad swaps and row rotations move data between lanes of
// a 16-lane row inside the VALU instruction, then v_readlane combines the four rows (LDS-based
// lane shuffles cost an LDS round trip per step).
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_ROR = 0x120;  // + rotation 1..15 within the row

// sum over each 16-lane row; every lane of the row ends with the row total
__device__ __forceinline__ int row_sum_i32(int v) {
  v += dpp_mov<DPP_QUAD_XOR1>(v);
  v += dpp_mov<DPP_QUAD_XOR2>(v);
  v += dpp_mov<DPP_ROW_ROR + 4>(v);
  v += dpp_mov<DPP_ROW_ROR + 8>(v);
  return v;
}
__device__ __forceinline__ int row_max_i32(int v) {
  v = max(v, dpp_mov<DPP_QUAD_XOR1>(v));
  v = max(v, dpp_mov<DPP_QUAD_XOR2>(v));
  v = max(v, dpp_mov<DPP_ROW_ROR + 4>(v));
  v = max(v, dpp_mov<DPP_ROW_ROR + 8>(v));
  return v;
}
__device__ __forceinline__ int rows4(int v, bool is_max) {
  const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return is_max ? max(max(a, b), max(c, d)) : a + b + c + d;
}
__device__ __forceinline__ int wave_sum_i32(int v) { return rows4(row_sum_i32(v), false); }
__device__ __forceinline__ int wave_max_i32(int v) { return rows4(row_max_i32(v), true); }

// sum of per-lane values below 2^48 (split into two 24-bit halves: each half-sum fits int32)
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)wave_sum_i32((int)(v & 0xFFFFFFu));
  const uint32_t hi = (uint32_t)wave_sum_i32((int)(v >> 24));
  return ((uint64_t)hi << 24) + lo;
}

// sum over aligned groups of G lanes (G in 4..64); the result is valid in the group's first lane
template <int G>
__device__ __forceinline__ int group_sum_i32(int v) {
  static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
  if constexpr (G <= 8) {
    v += dpp_mov<DPP_QUAD_XOR1>(v);
    v += dpp_mov<DPP_QUAD_XOR2>(v);
    if constexpr (G == 8) v += dpp_mov<DPP_HALF_MIRROR>(v);
    return v;
  } else {
    v = row_sum_i32(v);
    if constexpr (G == 16) return v;
    const int a = __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16);
    const int b = __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
    if constexpr (G == 64) return a + b;
    return (threadIdx.x & 32) ? b : a;
  }
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

// Branch-free operand loads: buffer loads (buffer_load_dword*) over a wave-uniform base and
// byte range.  An offset at or past the range reads zeros without touching memory, so a prologue
// can issue every load with no per-lane branch.  (A load inside a branch whose value is used in
// the branch makes the compiler wait there for every load issued before it: the counter of
// outstanding loads drains in issue order.)
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t LD_OOB = 0xFFFFFF00u;  // an offset past every range used here (< 2^31 bytes)

__device__ __forceinline__ Rsrc rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, base ? (int)(uint32_t)bytes : 0, 0x00020000);
}
__device__ __forceinline__ v4i ld16(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ v2i ld8(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ int32_t ld4(Rsrc r, uint32_t off) {
  return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ int32_t ld2s(Rsrc r, uint32_t off) {
  return (int32_t)(int16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
// keeps the loads of one prefetch group ahead of the next group's in issue order, and the code
// consuming a group behind every later group's issue: a wait for a group then leaves the later
// groups in flight
__device__ __forceinline__ void issue_fence() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
// the device decode position, read through the scalar cache (an earlier launch wrote it; the
// launch boundary makes it visible)
__device__ __forceinline__ int load_pos(const int32_t* pos_dev, int pos) {
  if (!pos_dev) return pos;
  return *(const __attribute__((address_space(4))) int32_t*)pos_dev;
}
// Touch every 64-byte line of the kernel arguments with one scalar load and wait once.  The
// compiler issues its argument loads lazily, between dependent steps, and each first touch of a
// line would cost a memory round trip (every graph launch has its own argument buffer); after
// this they hit the scalar cache.
template <int BYTES>
__device__ __forceinline__ void kernarg_warm() {
  static_assert(BYTES <= 768, "at most 12 argument lines");
  auto kp = __builtin_amdgcn_kernarg_segment_ptr();
  int d[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 12; ++i)
    if (64 * i < BYTES) __asm__ volatile("s_load_dword %0, %1, %2" : "=s"(d[i]) : "s"(kp), "i"(64 * i));
  // the loaded words are inputs of the wait so that they occupy distinct registers
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::"s"(d[0]), "s"(d[1]), "s"(d[2]), "s"(d[3]), "s"(d[4]), "s"(d[5]), "s"(d[6]),
                   "s"(d[7]), "s"(d[8]), "s"(d[9]), "s"(d[10]), "s"(d[11])
                   : "memory");
}
// wave index as a scalar (uniform) value, so per-wave buffer descriptors stay in SGPRs
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ int32_t lo16(int w) { return (int32_t)(int16_t)(w & 0xFFFF); }
__device__ __forceinline__ int32_t hi16(int w) { return (int32_t)(int16_t)((uint32_t)w >> 16); }
__device__ __forceinline__ int pack16(int64_t a, int64_t b) {
  return (int)(((uint32_t)(uint16_t)(int16_t)a) | ((uint32_t)(uint16_t)(int16_t)b << 16));
}

// RMSNorm reciprocal and one output value (golden.py:124-132)
__device__ __forceinline__ uint32_t rms_inv(uint64_t ss, uint32_t eps_t, uint32_t C) {
  const uint64_t tt = ss + eps_t;  // < 2^48: the host bounds K so that K * 2^30 + 2^32 < 2^48
  const uint32_t r = isqrt48(tt);
  const uint32_t d = r > 1 ? r : 1u;
  const uint32_t inv = C / d;  // C < 2^32: the quotient already fits u32
  return inv > 65535u ? 65535u : inv;
}

__device__ __forceinline__ int16_t rms_apply(int32_t x, int32_t g, uint32_t inv, int sh) {
  return (int16_t)sat16(rshr((int64_t)(x * g) * (int64_t)inv, sh));
}
// rms_apply with the row's scale = inv * 2^-sh in double: x * g (i16 x i16, |x g| <= 2^30) times
// inv (< 2^16) is below 2^46, so x g * scale + 1/2 is exact (a multiple of 2^-(sh+1) below 2^52, or
// for sh > 52 a value in (0, 1) whose floor 0 is exact) and its floor is rshr(x g inv, sh)
__device__ __forceinline__ double rms_scale(uint32_t inv, int sh) { return __builtin_ldexp((double)inv, -sh); }
__device__ __forceinline__ int32_t rms_apply_d(int32_t x, int32_t g, double scale) {
  const double v = __builtin_floor(__builtin_fma((double)(x * g), scale, 0.5));
  return (int32_t)__builtin_fmin(__builtin_fmax(v, -32768.0), 32767.0);
}

// argmax key: orders by value, then by lower index (larger key = better; golden.py:376-377 keeps
// the first maximum)
__device__ __forceinline__ uint64_t amax_key(int v, int64_t i) {
  return ((uint64_t)(uint32_t)(v + 32768) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

// int32 addition at device scope whose result is not used (a no-return vector atomic)
__device__ __forceinline__ void atomic_add_dev(int32_t* p, int32_t v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------
// RMSNorm + quant of rows (golden.py:124-137 + 119-120): parameters shared by the fused kernels and
// the split-K finish that normalises its output rows
// ---------------------------------------------------------------------------------------
struct NormQuant {
  const int16_t* x;
  const int16_t* gamma;
  int16_t* h_out;   // normalised rows (i16), written by workgroup 0
  int8_t* hq_out;   // quantised rows (i8), written by workgroup 0
  int64_t ldx;      // row stride of x and of the outputs (elements)
  int64_t Mq;       // quant multiplier
  uint32_t eps_t, C;
  int sh_post, Sq, K;
  int prequant;     // rows already normalised + quantised into h_out/hq_out
};

constexpr int NORM_MAX_K = 1024;  // a row's sum of squares takes chunks lane and lane + 64

inline int fill_pre(NormQuant& pr, const llhip_norm_quant_desc& d) {
  if (d.K <= 0 || d.K % 16 || d.ldx < d.K || d.ldx % 8)
    return fail(-EINVAL, "fused rmsnorm: K must be a multiple of 16 and ldx of 8");
  if (d.K > NORM_MAX_K) return fail(-EINVAL, "fused rmsnorm: K=%lld above %d", (long long)d.K, NORM_MAX_K);
  if (!u32_ok(d.eps_t) || !u32_ok(d.C) || !shift_ok(d.sh_post) || !u32_ok(d.Mq) || !shift_ok(d.Sq))
    return fail(-EINVAL, "fused rmsnorm/quant parameter out of range");
  if (d.K >= (int64_t)((1ull << 48) - (1ull << 32)) >> 30) return fail(-ERANGE, "isqrt48 input out of range");
  if ((uintptr_t)d.x % 16 || (uintptr_t)d.gamma % 16 || (d.h_out && (uintptr_t)d.h_out % 16) ||
      (d.hq_out && (uintptr_t)d.hq_out % 8))
    return fail(-EINVAL, "fused rmsnorm: misaligned operands");
  pr.x = static_cast<const int16_t*>(d.x);
  pr.gamma = static_cast<const int16_t*>(d.gamma);
  pr.h_out = static_cast<int16_t*>(d.h_out);
  pr.hq_out = static_cast<int8_t*>(d.hq_out);
  pr.ldx = d.ldx;
  pr.Mq = d.Mq;
  pr.eps_t = (uint32_t)d.eps_t;
  pr.C = (uint32_t)d.C;
  pr.sh_post = (int)d.sh_post;
  pr.Sq = (int)d.Sq;
  pr.K = (int)d.K;
  pr.prequant = d.prequant ? 1 : 0;
  if (pr.prequant && !d.hq_out) return fail(-EINVAL, "fused rmsnorm: prequant needs the quantised rows (hq_out)");
  return 0;
}

// ---------------------------------------------------------------------------------------
// misc
// ---------------------------------------------------------------------------------------
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Layout of the shared workspace (llhip_workspace_bytes(), zero-filled by the caller once).
// The greedy region must be zero on entry and every kernel leaves it zeroed again; the scratch
// region (GEMM split-K planes, split-context attention partials) is written in full before it is
// read within one call, so its contents between calls never matter.
constexpr int64_t WS_GREEDY = 5 << 20;         // uint64 best key + uint32 arrival counter
constexpr int64_t WS_SCRATCH = 8 << 20;
constexpr int64_t WS_SCRATCH_BYTES = 24 << 20;

int current_cu_count();

}  // namespace llhip
