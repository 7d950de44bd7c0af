// A device for the reference accelerator's instruction set (docs/ISA.md, binary version 2) on the
// GPU: the llaccel::Device contract of runtime/include/llaccel/device.h:15-29 with the semantics of
// the functional simulator runtime/src/funcsim.cpp.
//
// DRAM and the 1 MiB SRAM are device buffers.  run() walks the simulator's issue model on the host
// (funcsim.cpp:41-107: in-order issue into four engine queues, semaphores; the sequential policy
// executes every instruction right after it issues, an interleave seed picks random legal orders with
// the simulator's own generator), checks each instruction as the simulator does (same conditions, same
// messages), accumulates the same performance counters (functions of the operands and POS only) and
// enqueues the instruction's kernels on one stream: DMA and KV_WRITE as strided copies, GEMM as one
// kernel over the SRAM weight tiles, the VEC ops and ATTN through the datapath's own kernels.
// Data-dependent faults (an invalid requant table entry) set a device status flag.  The copies of the
// DMA and KV_WRITE instructions read it and write nothing once it is set, so no DMA or KV_WRITE after
// the failing GEMM changes memory, as in the simulator, which stops at that GEMM (funcsim.cpp:239);
// the host reads the flag when the program drains and when a later instruction fails, and then
// reports the simulator's message.  A DMA or KV_WRITE that fails at a row first writes the rows
// before it, as the simulator does.  After a failed run DRAM is the simulator's; SRAM written by the
// failed instruction (a GEMM's valid columns, ROPE/ATTN rows before a failing row, which the device
// does not write) and by VEC/GEMM/ATTN instructions after an invalid requant entry may differ.
#include <array>
#include <cstring>
#include <deque>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {
namespace {

constexpr uint32_t kSram = 1u << 20, kInstr = 64, kNumSem = 32, kTM = 16, kTMax = 4096, kBeat = 64, kQueueDepth = 8;
constexpr uint8_t kNoSem = 0xFF;
constexpr uint64_t kMaxInstr = 50000000;
constexpr uint64_t kDramPad = 64 << 10;  // zero bytes past the logical DRAM size (whole-tile reads)
enum Op : uint8_t {
  OP_NOP = 0x00, OP_HALT = 0x01, OP_DMA_LOAD = 0x10, OP_DMA_STORE = 0x11, OP_GEMM = 0x20, OP_RMSNORM = 0x30,
  OP_ROPE = 0x31, OP_SILU = 0x32, OP_MUL = 0x33, OP_ADD = 0x34, OP_QUANT = 0x35, OP_ATTN = 0x40, OP_KV_WRITE = 0x41,
};
// performance counter indices (include/llaccel/isa.h:133-141)
enum Perf {
  P_CYCLES = 0, P_INSTR_ISSUED, P_CP_STALL_WAIT, P_CP_STALL_QFULL, P_CP_STALL_FETCH, P_GEMM_BUSY, P_GEMM_MAC,
  P_GEMM_SRAM_STALL, P_GEMM_EPI, P_VEC_BUSY, P_VEC_SRAM_STALL, P_ATTN_BUSY, P_ATTN_SRAM_STALL, P_ATTN_MAC,
  P_DMA_BUSY, P_DMA_SRAM_STALL, P_DMA_DRAM_WAIT, P_SRAM_RD, P_SRAM_WR, P_DRAM_RD, P_DRAM_WR, P_GEMM_IDLE,
  P_VEC_IDLE, P_ATTN_IDLE, P_ATTN_DRAM_WAIT, P_ATTN_DRAM_RD, P_ATTN_DRAM_WR, P_NUM
};
static_assert(P_NUM == LLHIP_DEV_NUM_PERF, "27 performance counters");

const char* op_name(uint8_t op) {
  switch (op) {
    case OP_NOP: return "NOP";
    case OP_HALT: return "HALT";
    case OP_DMA_LOAD: return "DMA_LOAD";
    case OP_DMA_STORE: return "DMA_STORE";
    case OP_GEMM: return "GEMM";
    case OP_RMSNORM: return "VEC_RMSNORM";
    case OP_ROPE: return "VEC_ROPE";
    case OP_SILU: return "VEC_SILU";
    case OP_MUL: return "VEC_MUL";
    case OP_ADD: return "VEC_ADD";
    case OP_QUANT: return "VEC_QUANT";
    case OP_ATTN: return "ATTN";
    case OP_KV_WRITE: return "KV_WRITE";
  }
  return "?";
}
int engine_of(uint8_t op) { return op < 0x10 ? 0 : op < 0x20 ? 1 : op < 0x30 ? 2 : op < 0x40 ? 3 : 4; }

std::string hex(uint64_t v) {
  char b[32];
  std::snprintf(b, sizeof b, "%llx", (unsigned long long)v);
  return b;
}
[[noreturn]] void bad(const std::string& m) { throw std::runtime_error(m); }
void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) bad(std::string(what) + ": " + hipGetErrorString(e));
}
void rc_ok(int rc) {
  if (rc) bad(llhip_last_error());
}

// ---- kernels ----------------------------------------------------------------------------
// rows x bytes strided copy; 16-byte units when every address and stride allows it
// gate: a status flag; once it is set the copy writes nothing (NULL: always copy)
__global__ void copy_rows16(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, uint32_t rows, uint32_t units,
                            uint64_t ss, uint64_t ds, const int32_t* gate) {
  if (gate && *gate) return;
  const uint64_t n = (uint64_t)rows * units;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t r = i / units, u = i % units;
    *reinterpret_cast<uint4*>(dst + r * ds + 16 * u) = *reinterpret_cast<const uint4*>(src + r * ss + 16 * u);
  }
}
__global__ void copy_rows8(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, uint32_t rows, uint32_t bytes,
                           uint64_t ss, uint64_t ds, const int32_t* gate) {
  if (gate && *gate) return;
  const uint64_t n = (uint64_t)rows * bytes;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t r = i / bytes, b = i % bytes;
    dst[r * ds + b] = src[r * ss + b];
  }
}
// up to kBatch independent aligned copies in one launch (blockIdx.y = copy): consecutive DMA
// instructions that neither read nor write what another one of the batch writes
constexpr int kBatch = 8;
struct CopyBatch {
  uint8_t* dst[kBatch];
  const uint8_t* src[kBatch];
  uint32_t rows[kBatch], units[kBatch];
  uint64_t ss[kBatch], ds[kBatch];
  const int32_t* gate;
};
__global__ void copy_batch16(CopyBatch b) {
  if (b.gate && *b.gate) return;
  const int c = blockIdx.y;
  const uint32_t units = b.units[c];
  const uint64_t n = (uint64_t)b.rows[c] * units;
  uint8_t* dst = b.dst[c];
  const uint8_t* src = b.src[c];
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t r = i / units, u = i % units;
    *reinterpret_cast<uint4*>(dst + r * b.ds[c] + 16 * u) = *reinterpret_cast<const uint4*>(src + r * b.ss[c] + 16 * u);
  }
}
// destination rows that overlap each other: rows in order, one workgroup (later rows win)
__global__ void copy_rows_ordered(uint8_t* dst, const uint8_t* src, uint32_t rows, uint32_t bytes, uint64_t ss,
                                  uint64_t ds, const int32_t* gate) {
  if (gate && *gate) return;
  for (uint32_t r = 0; r < rows; ++r) {
    for (uint32_t b = threadIdx.x; b < bytes; b += blockDim.x) dst[r * ds + b] = src[r * ss + b];
    __syncthreads();
  }
}
// GEMM straight from the SRAM weight tiles, M <= 16 (funcsim.cpp:192-241): one workgroup per
// 16-column tile nt.  Tile (nt, kt) holds rows nt*16..+16 x columns kt*16..+16 of W as 16 rows of
// 16 bytes; thread t takes row n = t % 16 of tiles kt = t/16, t/16 + 16, ... (16-byte loads) and
// dot products them with the A rows' matching 16 bytes; the 16 partial sums of each (row, column)
// are added through LDS, and thread t = m*16 + n applies the bias, requant and epilogue of output
// (m, nt*16 + n).  A requant entry outside M_n >= 0, S_n in [0, 63] sets status flag 1 and leaves
// the column unwritten.
struct IsaGemm {
  const int8_t* A;
  const uint8_t* W;
  const int32_t* rq;
  const int32_t* bias;  // or null
  const int16_t* aux;   // resadd / mul, or null
  void* out;
  int32_t* status;
  uint32_t M, N, K, Mi;
  int mode, out_i8, aux_shift, Si, sh;
};
__global__ __launch_bounds__(256) void isa_gemm(IsaGemm g) {
  __shared__ int32_t part[16][16][17];  // [k group][row][column]
  const uint32_t nt = blockIdx.x, t = threadIdx.x, n = t & 15, q = t >> 4;
  const uint32_t KT = g.K / 16;
  int32_t acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0;
#pragma unroll 2
  for (uint32_t kt = q; kt < KT; kt += 16) {
    const int4 w = *reinterpret_cast<const int4*>(g.W + ((uint64_t)nt * KT + kt) * 256 + n * 16);
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if (m < (int)g.M) {
        const int4 a = *reinterpret_cast<const int4*>(g.A + (uint64_t)m * g.K + kt * 16);
        int32_t s = acc[m];
        s = __builtin_amdgcn_sdot4(a.x, w.x, s, false);
        s = __builtin_amdgcn_sdot4(a.y, w.y, s, false);
        s = __builtin_amdgcn_sdot4(a.z, w.z, s, false);
        acc[m] = __builtin_amdgcn_sdot4(a.w, w.w, s, false);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) part[q][m][n] = acc[m];
  __syncthreads();
  const uint32_t m = t >> 4;
  if (m >= g.M) return;
  int32_t sum = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) sum += part[k][m][n];
  const uint32_t ch = nt * 16 + n;
  const int32_t Mn = g.rq[2 * ch], Sn = g.rq[2 * ch + 1];
  if (Mn < 0 || Sn < 0 || Sn > 63) {
    atomicOr(g.status, 1);
    return;
  }
  const int64_t v = (int64_t)sum + (g.bias ? g.bias[ch] : 0);
  const uint64_t o = (uint64_t)m * g.N + ch;
  if (g.out_i8) {
    static_cast<int8_t*>(g.out)[o] = (int8_t)sat8(mulshift(v, Mn, Sn));
    return;
  }
  const int64_t tq = sat16(mulshift(v, Mn, Sn));
  int64_t y = tq;
  if (g.mode == 1)
    y = sat16(tq + g.aux[o]);
  else if (g.mode == 2)
    y = silu16(tq, g.Mi, g.Si, g.sh);
  else if (g.mode == 3)
    y = sat16(rshr(tq * g.aux[o], g.aux_shift));
  static_cast<int16_t*>(g.out)[o] = (int16_t)y;
}
// RoPE rows p = pos + m of the SRAM table [cos D/2][sin D/2] (row stride `stride` bytes) gathered
// into cos/sin [M][D/2]
__global__ void gather_rope(const uint8_t* __restrict__ sram, uint32_t table, uint32_t stride, uint32_t pos,
                            uint32_t M, uint32_t D, int16_t* __restrict__ cs, int16_t* __restrict__ sn) {
  const uint32_t h = D / 2;
  for (uint32_t i = threadIdx.x; i < M * D; i += blockDim.x) {
    const uint32_t m = i / D, j = i % D;
    const uint64_t a = (uint64_t)table + (uint64_t)(pos + m) * stride + 2ull * j;
    const int16_t v = (int16_t)(sram[a] | (sram[a + 1] << 8));
    if (j < h)
      cs[m * h + j] = v;
    else
      sn[m * h + j - h] = v;
  }
}
// KV_WRITE: src [M][Hkv*D] -> base + kvh*stride + (pos+m)*D (funcsim.cpp:390-398)
__global__ void kv_rows(uint8_t* __restrict__ dram, const uint8_t* __restrict__ src, uint64_t base, uint32_t M,
                        uint32_t Hkv, uint32_t D, uint64_t stride, uint32_t pos, const int32_t* gate) {
  if (*gate) return;
  const uint64_t n = (uint64_t)M * Hkv * D;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t d = i % D, r = i / D, kvh = r % Hkv, m = r / Hkv;
    dram[base + kvh * stride + (pos + m) * D + d] = src[i];
  }
}

unsigned grid_for(uint64_t n) { return (unsigned)std::min<uint64_t>(std::max<uint64_t>(ceil_div((int64_t)n, 256), 1), 4096); }

bool overlap(uint64_t a, uint64_t an, uint64_t b, uint64_t bn) { return an && bn && a < b + bn && b < a + an; }

}  // namespace

struct Device {
  uint8_t* dram = nullptr;
  uint64_t cap = 0, size = 0;  // allocation (without the pad) and the simulator's DRAM size
  uint8_t* sram = nullptr;
  uint8_t* scratch = nullptr;  // results of ops whose output aliases an input, copied back after
  int16_t* rope_tab = nullptr;
  void* ws = nullptr;
  int32_t* status = nullptr;
  hipStream_t stream = nullptr;
  bool fusion = false;
  bool rq_unchecked = false;  // a GEMM was enqueued since the status flag was last read
  uint32_t seed = 0;  // 0: sequential policy; else the simulator's random legal interleaving
  uint32_t pos = 0;
  uint64_t perf[P_NUM] = {};
  uint32_t sem[kNumSem] = {};

  ~Device() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (void* p : {(void*)dram, (void*)sram, (void*)scratch, (void*)rope_tab, ws, (void*)status})
      if (p) (void)hipFree(p);
    if (stream) (void)hipStreamDestroy(stream);
  }

  void init(uint64_t dram_bytes, bool epilogue_fusion) {
    fusion = epilogue_fusion;
    hip_ok(hipStreamCreate(&stream), "hipStreamCreate");
    hip_ok(hipMalloc(&sram, kSram), "hipMalloc");
    hip_ok(hipMalloc(&scratch, kSram), "hipMalloc");
    hip_ok(hipMalloc(&rope_tab, 2 * kTM * 128 * sizeof(int16_t)), "hipMalloc");
    hip_ok(hipMalloc(&ws, (size_t)llhip_workspace_bytes()), "hipMalloc");
    hip_ok(hipMalloc(&status, 4), "hipMalloc");
    hip_ok(hipMemset(sram, 0, kSram), "hipMemset");
    hip_ok(hipMemset(ws, 0, (size_t)llhip_workspace_bytes()), "hipMemset");
    hip_ok(hipMemset(status, 0, 4), "hipMemset");
    grow(std::max<uint64_t>(dram_bytes, 1u << 20));
  }

  // the simulator's ensureDram: the DRAM grows (zero-filled) to n bytes
  void grow(uint64_t n) {
    if (n <= size) return;
    if (n > cap) {
      flush();
      const uint64_t ncap = std::max<uint64_t>((n + (1u << 20) - 1) & ~uint64_t((1u << 20) - 1), 2 * cap);
      uint8_t* nd = nullptr;
      hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
      hip_ok(hipMalloc(&nd, ncap + kDramPad), "hipMalloc (DRAM)");
      hip_ok(hipMemset(nd, 0, ncap + kDramPad), "hipMemset");
      if (dram) {
        hip_ok(hipMemcpy(nd, dram, size, hipMemcpyDeviceToDevice), "hipMemcpy");
        hip_ok(hipFree(dram), "hipFree");
      }
      dram = nd;
      cap = ncap;
    }
    size = n;  // bytes past the old size are zero: nothing is ever written beyond `size`
  }

  void write(uint64_t addr, const void* src, uint64_t n) {
    if (addr > UINT64_MAX - n) bad("dramWrite address overflow");
    grow(addr + n);
    hip_ok(hipMemcpyAsync(dram + addr, src, n, hipMemcpyHostToDevice, stream), "hipMemcpyAsync");
    hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }
  void read(uint64_t addr, void* dst, uint64_t n) {
    if (addr > size || n > size - addr) bad("dramRead out of range");
    hip_ok(hipMemcpyAsync(dst, dram + addr, n, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }

  // ---- checks (funcsim.cpp:124-132) ----
  static void chk(uint64_t addr, uint64_t n, const char* what) {
    if (addr + n > kSram) bad(std::string("SRAM access out of range in ") + what + " @0x" + hex(addr));
  }
  void chk_dram(uint64_t addr, uint64_t n, const char* what) const {
    if (addr > size || n > size - addr || addr > UINT32_MAX || n > uint64_t(UINT32_MAX) + 1 - addr)
      bad(std::string("DRAM access out of range in ") + what + " @0x" + hex(addr));
  }
  // SRAM operands of the datapath kernels: 16-byte aligned (docs/ISA.md "Opcodes")
  static void aligned(uint64_t addr, const char* what) {
    if (addr % 16) bad(std::string("SRAM operand not 16-B aligned in ") + what + " @0x" + hex(addr));
  }
  // An output that aliases an input: exactly (dst == src, the simulator's element-by-element loops
  // read each element before writing it) -> computed into scratch and copied back; any other
  // overlap would see partially updated inputs in the simulator's order -> rejected.
  static bool alias(uint64_t dst, uint64_t dn, uint64_t src, uint64_t sn, const char* what) {
    if (!overlap(dst, dn, src, sn)) return false;
    if (dst != src) bad(std::string("overlapping operands in ") + what);
    return true;
  }

  // queued DMA copies: offsets (the DRAM may move when it grows) and the byte ranges they touch
  struct Pending {
    bool load;
    uint64_t sram_off, dram_off, rows, bytes, ss, ds;
    uint64_t span(uint64_t stride) const { return (rows - 1) * stride + bytes; }
  };
  std::vector<Pending> pend;
  // the DRAM range of the fetched instruction window: a DRAM write into it refetches the window,
  // so a program that stores over its own later instructions runs what it stored, as in the simulator
  uint64_t win_lo = 0, win_hi = 0;
  bool win_stale = false;
  void dram_written(uint64_t lo, uint64_t n) {
    if (overlap(lo, n, win_lo, win_hi - win_lo)) win_stale = true;
  }

  void flush() {
    if (pend.empty()) return;
    CopyBatch b{};
    uint64_t most = 0;
    for (size_t i = 0; i < pend.size(); ++i) {
      const Pending& q = pend[i];
      b.dst[i] = q.load ? sram + q.sram_off : dram + q.dram_off;
      b.src[i] = q.load ? dram + q.dram_off : sram + q.sram_off;
      b.rows[i] = (uint32_t)q.rows;
      b.units[i] = (uint32_t)(q.bytes / 16);
      b.ss[i] = q.ss;
      b.ds[i] = q.ds;
      most = std::max<uint64_t>(most, q.rows * q.bytes / 16);
    }
    const int n = (int)pend.size();
    pend.clear();
    b.gate = status;
    hipLaunchKernelGGL(copy_batch16, dim3(grid_for(most), n), dim3(256), 0, stream, b);
    hip_ok(hipGetLastError(), "kernel launch");
  }

  // a DMA joins the batch when it is aligned, its rows do not overlap, and it neither writes what a
  // queued copy reads or writes nor reads what a queued copy writes
  void queue_dma(bool load, uint64_t sramA, uint64_t dramA, uint64_t rows, uint64_t bytes, uint64_t ss, uint64_t ds) {
    if (!rows || !bytes) return;
    Pending q{load, sramA, dramA, rows, bytes, ss, ds};
    const bool ok = (rows == 1 || ds >= bytes) && ((uintptr_t)dram | sramA | dramA | ss | ds | bytes) % 16 == 0;
    if (!ok) {
      flush();
      if (load)
        copy(sram + sramA, dram + dramA, (uint32_t)rows, (uint32_t)bytes, ss, ds, status);
      else
        copy(dram + dramA, sram + sramA, (uint32_t)rows, (uint32_t)bytes, ss, ds, status);
      return;
    }
    // ranges: [lo, lo + span) in SRAM (sram side) or DRAM (dram side)
    const uint64_t q_dst_lo = load ? sramA : dramA, q_src_lo = load ? dramA : sramA;
    const uint64_t q_dst_n = q.span(ds), q_src_n = q.span(ss);
    for (const Pending& o : pend) {
      const uint64_t o_dst_lo = o.load ? o.sram_off : o.dram_off, o_src_lo = o.load ? o.dram_off : o.sram_off;
      const uint64_t o_dst_n = o.span(o.ds), o_src_n = o.span(o.ss);
      // same memory when both destinations are SRAM (both loads) or both DRAM (both stores), etc.
      const bool dd = (o.load == load) && overlap(q_dst_lo, q_dst_n, o_dst_lo, o_dst_n);
      const bool ds_ = (o.load != load) && overlap(q_dst_lo, q_dst_n, o_src_lo, o_src_n);
      const bool sd = (o.load != load) && overlap(q_src_lo, q_src_n, o_dst_lo, o_dst_n);
      if (dd || ds_ || sd) {
        flush();
        break;
      }
    }
    pend.push_back(q);
    if ((int)pend.size() == kBatch) flush();
  }

  // gate: the status flag for the copies of DMA instructions, NULL for the copy-back of an op's
  // in-place result
  void copy(uint8_t* dst, const uint8_t* src, uint32_t rows, uint32_t bytes, uint64_t ss, uint64_t ds,
            const int32_t* gate = nullptr) {
    if (!rows || !bytes) return;
    if (rows > 1 && ds < bytes) {
      hipLaunchKernelGGL(copy_rows_ordered, dim3(1), dim3(256), 0, stream, dst, src, rows, bytes, ss, ds, gate);
    } else if (((uintptr_t)dst | (uintptr_t)src | ss | ds | bytes) % 16 == 0) {
      hipLaunchKernelGGL(copy_rows16, dim3(grid_for((uint64_t)rows * bytes / 16)), dim3(256), 0, stream, dst, src, rows,
                         bytes / 16, ss, ds, gate);
    } else {
      hipLaunchKernelGGL(copy_rows8, dim3(grid_for((uint64_t)rows * bytes)), dim3(256), 0, stream, dst, src, rows, bytes,
                         ss, ds, gate);
    }
    hip_ok(hipGetLastError(), "kernel launch");
  }

  // the range checks of DMA row r (funcsim.cpp:171-184)
  void row_check(uint32_t r, bool load, uint32_t sramA, uint32_t dramA, uint32_t rowBytes, uint32_t srcStride,
                 uint32_t dstStride) const {
    if (load) {
      const uint64_t s = uint64_t(dramA) + uint64_t(r) * srcStride, d = uint64_t(sramA) + uint64_t(r) * dstStride;
      if (s + rowBytes > size) bad("DMA_LOAD source out of DRAM range");
      chk(d, rowBytes, "DMA_LOAD");
    } else {
      chk(uint64_t(sramA) + uint64_t(r) * srcStride, rowBytes, "DMA_STORE");
    }
  }

  // Reads the requant status flag once the work enqueued so far has run (when the program drains or
  // an instruction fails); raises the simulator's error if a GEMM met an invalid table entry
  // (funcsim.cpp:239).
  void requant_check() {
    if (!rq_unchecked) return;
    rq_unchecked = false;
    flush();
    int32_t st = 0;
    hip_ok(hipMemcpyAsync(&st, status, 4, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (st & 1) bad("invalid requantization table entry");
  }

  // ---- instructions ----
  void dma(const uint32_t* in, bool load) {
    const uint32_t sramA = in[2], dramA = in[3], rows = in[4], rowBytes = in[5], srcStride = in[6], dstStride = in[7];
    if (rowBytes % 16 || sramA % 16) bad("DMA row/addr not 16-B aligned");
    uint64_t beats = 0, sramReadBytes = 0;
    uint32_t r = 0;
    // a row that fails its check: the rows before it are copied first (funcsim.cpp:162-186 copies
    // row by row)
    try {
      for (; r < rows; ++r) row_check(r, load, sramA, dramA, rowBytes, srcStride, dstStride);
    } catch (...) {
      if (r) queue_dma(load, sramA, dramA, r, rowBytes, srcStride, dstStride);
      throw;
    }
    for (r = 0; r < rows; ++r) {  // funcsim.cpp:162-186
      const uint64_t dramRow = uint64_t(dramA) + uint64_t(r) * (load ? srcStride : dstStride);
      beats += rowBytes ? ((dramRow % 64) + rowBytes + 63) / 64 : 0;
      if (!load) {
        uint64_t copied = 0;
        while (copied < rowBytes) {
          const uint64_t useful = std::min<uint64_t>(64 - ((dramRow + copied) % 64), rowBytes - copied);
          const uint64_t source = uint64_t(sramA) + uint64_t(r) * srcStride + copied;
          sramReadBytes += ((source % 64 + useful + 63) / 64) * 64;
          copied += useful;
        }
      }
      if (!load) {
        const uint64_t d = uint64_t(dramA) + uint64_t(r) * dstStride;
        grow(d + rowBytes);
        dram_written(d, rowBytes);
      }
    }
    const uint64_t bytes = uint64_t(rows) * rowBytes;
    perf[load ? P_SRAM_WR : P_SRAM_RD] += load ? bytes : sramReadBytes;
    perf[load ? P_DRAM_RD : P_DRAM_WR] += beats * 64;
    perf[P_DMA_BUSY] += beats;
    queue_dma(load, sramA, dramA, rows, rowBytes, srcStride, dstStride);
  }

  void gemm(const uint32_t* in) {
    const uint32_t a = in[2], w = in[3], out = in[4], rq = in[5], bias = in[6], aux = in[7];
    const uint32_t M = in[8], N = in[9], K = in[10], ep = in[11], siluMi = in[12], siluSi = in[13] & 0xFF,
                   siluSh = (in[13] >> 8) & 0xFF;
    const bool hasBias = (in[0] >> 8) & 1;
    const uint32_t mode = ep & 0xF;
    const bool outI8 = (ep >> 4) & 1;
    const uint32_t auxShift = (ep >> 8) & 0xFF;
    if (M == 0 || M > kTM || N % 16 || K % 16 || N == 0 || K == 0) bad("GEMM bad shape");
    if (w % 256) bad("GEMM weight address not 256-B aligned");
    if (outI8 && mode != 0) bad("GEMM i8 output with epilogue");
    if (mode != 0 && !fusion) bad("GEMM epilogue used on a target without EPILOGUE_FUSION");
    const uint32_t NT = N / 16, KT = K / 16, outRow = outI8 ? N : 2 * N;
    chk(a, uint64_t(M) * K, "GEMM A");
    chk(w, uint64_t(NT) * KT * 256, "GEMM W");
    chk(rq, uint64_t(N) * 8, "GEMM rq");
    chk(out, uint64_t(M) * outRow, "GEMM out");
    if (hasBias) chk(bias, uint64_t(N) * 4, "GEMM bias");
    const bool useAux = mode == 1 || mode == 3;
    if (useAux) chk(aux, uint64_t(M) * 2 * N, "GEMM aux");
    if (mode > 3) bad("GEMM bad epilogue mode");
    for (uint32_t x : {a, out, rq}) aligned(x, "GEMM");
    if (hasBias) aligned(bias, "GEMM");
    if (useAux) aligned(aux, "GEMM");
    const uint64_t on = uint64_t(M) * outRow;
    if (overlap(out, on, a, uint64_t(M) * K) || overlap(out, on, w, uint64_t(NT) * KT * 256) ||
        overlap(out, on, rq, uint64_t(N) * 8) || (hasBias && overlap(out, on, bias, uint64_t(N) * 4)))
      bad("overlapping operands in GEMM");
    const bool inplace = useAux && alias(out, on, aux, uint64_t(M) * 2 * N, "GEMM");
    // counters of funcsim.cpp:202-239 in closed form
    perf[P_SRAM_RD] += uint64_t(NT) * KT * (256 + uint64_t(M) * 16) + uint64_t(NT) * (128 + (hasBias ? 64 : 0)) +
                       (useAux ? uint64_t(NT) * M * 32 : 0);
    perf[P_GEMM_MAC] += uint64_t(NT) * KT * M;
    perf[P_SRAM_WR] += uint64_t(NT) * M * (outI8 ? 16 : 32);
    perf[P_GEMM_EPI] += uint64_t(NT) * M;
    perf[P_GEMM_BUSY] += uint64_t(NT) * KT * (1 + M) + uint64_t(NT) * M;

    uint8_t* dst = inplace ? scratch : sram + out;
    IsaGemm g{reinterpret_cast<const int8_t*>(sram + a), sram + w, reinterpret_cast<const int32_t*>(sram + rq),
              hasBias ? reinterpret_cast<const int32_t*>(sram + bias) : nullptr,
              useAux ? reinterpret_cast<const int16_t*>(sram + aux) : nullptr, dst, status, M, N, K, siluMi,
              (int)mode, outI8 ? 1 : 0, (int)auxShift, (int)siluSi, (int)siluSh};
    hipLaunchKernelGGL(isa_gemm, dim3(NT), dim3(256), 0, stream, g);
    hip_ok(hipGetLastError(), "kernel launch");
    rq_unchecked = true;
    if (inplace) copy(sram + out, scratch, 1, (uint32_t)on, 0, 0);
  }

  void rmsnorm(const uint32_t* in) {
    const uint32_t src = in[2], gamma = in[3], dst = in[4], M = in[5], K = in[6], epsT = in[7], C = in[8], shPost = in[9];
    if (K % 16 || K == 0) bad("RMSNORM K not a multiple of 16");
    const uint64_t n = uint64_t(M) * K * 2;
    chk(src, n, "RMSNORM src");
    chk(gamma, uint64_t(K) * 2, "RMSNORM gamma");
    chk(dst, n, "RMSNORM dst");
    perf[P_SRAM_RD] += uint64_t(M) * (2 * K * 2 + K * 2);
    perf[P_SRAM_WR] += uint64_t(M) * K * 2;
    perf[P_VEC_BUSY] += uint64_t(M) * (2 * K / 16 + 24 + 32);
    if (!M) return;
    for (uint32_t x : {src, gamma, dst}) aligned(x, "VEC_RMSNORM");
    if (overlap(dst, n, gamma, uint64_t(K) * 2)) bad("overlapping operands in VEC_RMSNORM");
    const bool inplace = alias(dst, n, src, n, "VEC_RMSNORM");
    int16_t* y = reinterpret_cast<int16_t*>(inplace ? scratch : sram + dst);
    rc_ok(llhip_rmsnorm(reinterpret_cast<const int16_t*>(sram + src), M, K, K,
                        reinterpret_cast<const int16_t*>(sram + gamma), epsT, C, shPost, y, K, stream));
    if (inplace) copy(sram + dst, scratch, 1, (uint32_t)n, 0, 0);
  }

  void rope(const uint32_t* in) {
    const uint32_t src = in[2], dst = in[3], M = in[4], H = in[5], D = in[6], table = in[7], stride = in[8];
    if (D != 16 && D != 32 && D != 64 && D != 128 && D != 256) bad("ROPE bad D");
    if (M == 0 || M > kTM || H == 0 || H > 255 || pos >= kTMax || M > kTMax - pos || stride < 2 * D)
      bad("ROPE invalid row/head/context dimensions");
    const uint32_t row = H * D;
    const uint64_t n = uint64_t(M) * row * 2;
    chk(src, n, "ROPE src");
    chk(dst, n, "ROPE dst");
    for (uint32_t m = 0; m < M; ++m) chk(uint64_t(table) + uint64_t(pos + m) * stride, 2 * D, "ROPE table");
    perf[P_SRAM_RD] += uint64_t(M) * (row * 2 + H * 2 * D);
    perf[P_SRAM_WR] += uint64_t(M) * row * 2;
    perf[P_VEC_BUSY] += uint64_t(M) * H * (D / 2 / 16 + 1);
    aligned(src, "VEC_ROPE");
    aligned(dst, "VEC_ROPE");
    for (uint32_t m = 0; m < M; ++m)
      if (overlap(dst, n, uint64_t(table) + uint64_t(pos + m) * stride, 2 * D)) bad("overlapping operands in VEC_ROPE");
    const bool inplace = alias(dst, n, src, n, "VEC_ROPE");
    int16_t* cs = rope_tab;
    int16_t* sn = rope_tab + kTM * 128;
    hipLaunchKernelGGL(gather_rope, dim3(1), dim3(256), 0, stream, sram, table, stride, pos, M, D, cs, sn);
    hip_ok(hipGetLastError(), "kernel launch");
    int16_t* y = reinterpret_cast<int16_t*>(inplace ? scratch : sram + dst);
    rc_ok(llhip_rope(reinterpret_cast<const int16_t*>(sram + src), M, H, D, row, cs, sn, M, 0, nullptr, nullptr, y, row,
                     stream));
    if (inplace) copy(sram + dst, scratch, 1, (uint32_t)n, 0, 0);
  }

  // kind: 0 SILU(src,dst,count,Mi,Si,sh_out) 1 MUL(a,b,dst,count,sh) 2 ADD(a,b,dst,count,sh_b) 3 QUANT(src,dst,count,M,S)
  void elementwise(const uint32_t* in, int kind) {
    static const char* names[] = {"VEC_SILU", "VEC_MUL", "VEC_ADD", "VEC_QUANT"};
    if (kind == 0 || kind == 3) {
      const uint32_t src = in[2], dst = in[3], count = in[4], p0 = in[5], p1 = in[6], p2 = in[7];
      if (count % 16) bad("VEC count not a multiple of 16");
      const uint64_t dn = uint64_t(count) * (kind == 3 ? 1 : 2);
      chk(src, uint64_t(count) * 2, "VEC src");
      chk(dst, dn, "VEC dst");
      perf[P_SRAM_RD] += uint64_t(count) * 2;
      perf[P_SRAM_WR] += dn;
      perf[P_VEC_BUSY] += count / 16;
      if (!count) return;
      aligned(src, names[kind]);
      aligned(dst, names[kind]);
      // dst at or before src: the simulator's ascending loop reads every element before it is overwritten
      bool inplace = false;
      if (overlap(dst, dn, src, uint64_t(count) * 2)) {
        if (dst > src) bad(std::string("overlapping operands in ") + names[kind]);
        inplace = true;
      }
      uint8_t* y = inplace ? scratch : sram + dst;
      const int16_t* x = reinterpret_cast<const int16_t*>(sram + src);
      if (kind == 0)
        rc_ok(llhip_silu(x, count, p0, p1, p2, reinterpret_cast<int16_t*>(y), stream));
      else
        rc_ok(llhip_quant(x, count, p0, p1, reinterpret_cast<int8_t*>(y), stream));
      if (inplace) copy(sram + dst, scratch, 1, (uint32_t)dn, 0, 0);
    } else {
      const uint32_t a = in[2], b = in[3], dst = in[4], count = in[5], sh = in[6];
      if (count % 16) bad("VEC count not a multiple of 16");
      const uint64_t n = uint64_t(count) * 2;
      chk(a, n, "VEC a");
      chk(b, n, "VEC b");
      chk(dst, n, "VEC dst");
      perf[P_SRAM_RD] += uint64_t(count) * 4;
      perf[P_SRAM_WR] += n;
      perf[P_VEC_BUSY] += count / 16;
      if (!count) return;
      for (uint32_t x : {a, b, dst}) aligned(x, names[kind]);
      bool inplace = false;
      for (uint32_t s : {a, b})
        if (overlap(dst, n, s, n)) {
          if (dst > s) bad(std::string("overlapping operands in ") + names[kind]);
          inplace = true;
        }
      int16_t* y = reinterpret_cast<int16_t*>(inplace ? scratch : sram + dst);
      const int16_t* x0 = reinterpret_cast<const int16_t*>(sram + a);
      const int16_t* x1 = reinterpret_cast<const int16_t*>(sram + b);
      if (kind == 1)
        rc_ok(llhip_vmul(x0, x1, count, sh, y, stream));
      else
        rc_ok(llhip_vadd(x0, x1, count, sh, y, stream));
      if (inplace) copy(sram + dst, scratch, 1, (uint32_t)n, 0, 0);
    }
  }

  // DRAM beats of T key rows of D bytes from `base` (funcsim.cpp:364-369): one 64-byte beat per row,
  // D/16 when the row crosses a beat; periodic in t with period at most 4, so counted per period
  static uint64_t row_beats(uint64_t base, uint32_t T, uint32_t D) {
    uint64_t per[4], period = 0;
    for (uint32_t t = 0; t < 4; ++t) per[t] = ((base + uint64_t(t) * D) % kBeat + D > kBeat) ? D / 16 : 1;
    uint64_t full = 0;
    for (uint32_t t = 0; t < 4; ++t) full += per[t];
    period = uint64_t(T / 4) * full;
    for (uint32_t t = 0; t < T % 4; ++t) period += per[t];
    return period;
  }

  void attn(const uint32_t* in) {
    const uint32_t q = in[2], out = in[3], kbase = in[4], vbase = in[5], M = in[6], H = in[7], Hkv = in[8], D = in[9],
                   kvStride = in[10], Ms = in[11], Ss = in[12], Mo = in[13], So = in[14];
    if (D != 16 && D != 32 && D != 64 && D != 128 && D != 256) bad("ATTN bad D");
    if (M == 0 || M > kTM || H == 0 || H > 255 || Hkv == 0 || Hkv > 255 || H % Hkv)
      bad("ATTN invalid row/head dimensions");
    if (pos >= kTMax || M > kTMax - pos || uint64_t(pos + M) * D > kvStride || kvStride % 16 || kbase % 16 ||
        vbase % 16)
      bad("ATTN invalid context/DRAM cache stride");
    const uint32_t row = H * D, grp = H / Hkv;
    const uint64_t n = uint64_t(M) * row;
    chk(q, n, "ATTN q");
    chk(out, n, "ATTN out");
    const uint32_t Tmax = pos + M;
    for (uint32_t kvh = 0; kvh < Hkv; ++kvh) {  // the widest row's keys of every head group
      chk_dram(uint64_t(kbase) + uint64_t(kvh) * kvStride, uint64_t(Tmax) * D, "ATTN K");
      chk_dram(uint64_t(vbase) + uint64_t(kvh) * kvStride, uint64_t(Tmax) * D, "ATTN V");
    }
    if (kvStride % D) bad("ATTN kv_stride not a multiple of D is not supported by this device");
    for (uint32_t m = 0; m < M; ++m) {
      const uint32_t T = pos + m + 1;
      for (uint32_t h = 0; h < H; ++h) {
        const uint32_t kvh = h / grp;
        const uint64_t kb = uint64_t(kbase) + uint64_t(kvh) * kvStride, vb = uint64_t(vbase) + uint64_t(kvh) * kvStride;
        const uint64_t kvRead = (3 * row_beats(kb, T, D) + row_beats(vb, T, D)) * kBeat;
        perf[P_SRAM_RD] += D;
        perf[P_DRAM_RD] += kvRead;
        perf[P_ATTN_DRAM_RD] += kvRead;
        perf[P_SRAM_WR] += D;
        perf[P_ATTN_MAC] += 4ull * T;
        perf[P_ATTN_BUSY] += 7ull * T + 32;
      }
    }
    aligned(q, "ATTN");
    aligned(out, "ATTN");
    const bool inplace = alias(out, n, q, n, "ATTN");
    int8_t* o = reinterpret_cast<int8_t*>(inplace ? scratch : sram + out);
    const int pb = ((in[0] >> 8) & 2) ? 15 : 8;
    rc_ok(llhip_attention(reinterpret_cast<const int8_t*>(sram + q), M, H, Hkv, D, row, pos, nullptr, nullptr, 0,
                          reinterpret_cast<const int8_t*>(dram + kbase), reinterpret_cast<const int8_t*>(dram + vbase),
                          kvStride / D, Ms, Ss, Mo, So, pb, o, row, ws, stream));
    if (inplace) copy(sram + out, scratch, 1, (uint32_t)n, 0, 0);
  }

  void kv_write(const uint32_t* in) {
    const uint32_t src = in[2], base = in[3], M = in[4], Hkv = in[5], D = in[6], kvStride = in[7];
    if ((D != 16 && D != 32 && D != 64 && D != 128 && D != 256) || M == 0 || M > kTM || Hkv == 0 || Hkv > 255 ||
        pos >= kTMax || M > kTMax - pos || uint64_t(pos + M) * D > kvStride || kvStride % 16 || base % 16)
      bad("KV_WRITE invalid dimensions/DRAM cache stride");
    const uint32_t row = Hkv * D;
    chk(src, uint64_t(M) * row, "KV_WRITE src");
    for (uint32_t m = 0; m < M; ++m)
      for (uint32_t kvh = 0; kvh < Hkv; ++kvh) {
        const uint64_t d = uint64_t(base) + uint64_t(kvh) * kvStride + uint64_t(pos + m) * D;
        try {
          chk_dram(d, D, "KV_WRITE dst");
        } catch (...) {  // the (row, head) pairs before this one are written first (funcsim.cpp:388-398)
          if (m) kv_launch(src, base, m, Hkv, D, kvStride, pos);
          if (kvh) kv_launch(src + m * row, base, 1, kvh, D, kvStride, pos + m);
          throw;
        }
        dram_written(d, D);
        const uint64_t wr = ((d % kBeat + D > kBeat) ? D / 16 : 1) * kBeat;
        perf[P_DRAM_WR] += wr;
        perf[P_ATTN_DRAM_WR] += wr;
      }
    perf[P_SRAM_RD] += uint64_t(M) * row;
    perf[P_ATTN_BUSY] += uint64_t(M) * Hkv;
    kv_launch(src, base, M, Hkv, D, kvStride, pos);
  }

  // heads 0..Hkv-1 of M rows of `src` (row stride Hkv * D) into the cache rows p .. p+M-1
  void kv_launch(uint32_t src, uint32_t base, uint32_t M, uint32_t Hkv, uint32_t D, uint32_t kvStride, uint32_t p) {
    hipLaunchKernelGGL(kv_rows, dim3(grid_for(uint64_t(M) * Hkv * D)), dim3(256), 0, stream, dram, sram + src,
                       uint64_t(base), M, Hkv, D, uint64_t(kvStride), p, status);
    hip_ok(hipGetLastError(), "kernel launch");
  }

  void execute(const uint32_t* in) {
    const uint8_t op = in[0] & 0xFF;
    auto shift = [](uint32_t s) {
      if (s > 63) bad("shift outside [0,63]");
    };
    switch (op) {  // funcsim.cpp:131-138
      case OP_GEMM: shift((in[11] >> 8) & 0xFF); shift(in[13] & 255); shift((in[13] >> 8) & 255); break;
      case OP_RMSNORM: shift(in[9]); break;
      case OP_SILU: shift(in[6]); shift(in[7]); break;
      case OP_QUANT: case OP_ADD: case OP_MUL: shift(in[6]); break;
      case OP_ATTN: shift(in[12]); shift(in[14]); break;
      default: break;
    }
    if (op != OP_DMA_LOAD && op != OP_DMA_STORE) flush();
    switch (op) {
      case OP_DMA_LOAD: return dma(in, true);
      case OP_DMA_STORE: return dma(in, false);
      case OP_GEMM: return gemm(in);
      case OP_RMSNORM: return rmsnorm(in);
      case OP_ROPE: return rope(in);
      case OP_SILU: return elementwise(in, 0);
      case OP_MUL: return elementwise(in, 1);
      case OP_ADD: return elementwise(in, 2);
      case OP_QUANT: return elementwise(in, 3);
      case OP_ATTN: return attn(in);
      case OP_KV_WRITE: return kv_write(in);
      default: bad("unexpected opcode " + std::to_string(int(op)));
    }
  }

  // Fetches, checks and executes instructions from `pc` until HALT (funcsim.cpp:41-107).
  void run(uint32_t pc, uint32_t p) {
    pend.clear();
    try {
      run_program(pc, p);
    } catch (...) {
      try {
        flush();  // the DMAs before a failing instruction have happened, as in the simulator
      } catch (...) {
      }
      // an invalid requant entry met by an earlier GEMM is the error the simulator stopped at
      requant_check();
      throw;
    }
  }

  void run_program(uint32_t pc, uint32_t p) {
    std::memset(perf, 0, sizeof perf);
    std::memset(sem, 0, sizeof sem);
    pos = p;
    hip_ok(hipMemsetAsync(status, 0, 4, stream), "hipMemsetAsync");
    rq_unchecked = false;
    std::vector<uint32_t> window;  // instructions fetched from DRAM, 1024 at a time
    uint64_t wbase = 0, fetchPc = pc, issued = 0;
    win_lo = win_hi = 0;
    win_stale = false;
    // the engine queues (dma, gemm, vec, attn) of the simulator's issue model, funcsim.cpp:46-105:
    // each round the candidates are the non-empty queues' heads and, while not halted, issuing the
    // next instruction (its semaphore wait met and its queue not full); the sequential policy takes
    // the first queue head (so every instruction runs right after it issues), an interleave seed a
    // uniformly random candidate from the same generator and distribution as the simulator
    std::deque<std::array<uint32_t, 16>> queues[5];
    std::mt19937 rng(seed);
    bool halted = false;
    std::vector<int> cands;
    for (;;) {
      cands.clear();
      for (int e = 1; e <= 4; ++e)
        if (!queues[e].empty()) cands.push_back(e);
      std::array<uint32_t, 16> next{};
      if (!halted) {
        if (fetchPc + kInstr > size) bad("instruction fetch out of DRAM range");
        if (win_stale || window.empty() || fetchPc < wbase || fetchPc + kInstr > wbase + window.size() * 4) {
          flush();
          const uint64_t n = std::min<uint64_t>(1024 * kInstr, (size - fetchPc) / kInstr * kInstr);
          window.assign(n / 4, 0);
          wbase = fetchPc;
          win_lo = wbase;
          win_hi = wbase + n;
          win_stale = false;
          // ordered after every instruction enqueued so far: a program that stores over its own
          // later instructions sees them as the simulator does
          hip_ok(hipMemcpyAsync(window.data(), dram + fetchPc, n, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
          hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
        }
        std::memcpy(next.data(), window.data() + (fetchPc - wbase) / 4, sizeof next);
        const uint8_t op = next[0] & 0xFF, ws_ = (next[0] >> 16) & 0xFF, ss = (next[0] >> 24) & 0xFF;
        if ((ws_ != kNoSem && ws_ >= kNumSem) || (ss != kNoSem && ss >= kNumSem)) bad("invalid semaphore index");
        if (engine_of(op) == 0 && op != OP_NOP && op != OP_HALT) bad("invalid command processor opcode");
        const bool waitOk = ws_ == kNoSem || sem[ws_] >= next[1];
        const int eng = engine_of(op);
        if (waitOk && (eng == 0 || queues[eng].size() < kQueueDepth)) cands.push_back(0);
      }
      if (cands.empty()) {
        if (halted) break;  // every queue drained after HALT
        const uint8_t op = next[0] & 0xFF, ws_ = (next[0] >> 16) & 0xFF;
        bad("deadlock at pc=0x" + hex(fetchPc) + " (" + op_name(op) + " waits sem " + std::to_string(ws_) + " >= " +
            std::to_string(next[1]) + ", current " + std::to_string(ws_ == kNoSem ? 0 : sem[ws_]) + ")");
      }
      const int choice = seed == 0 ? cands[0]
                                   : cands[std::uniform_int_distribution<size_t>(0, cands.size() - 1)(rng)];
      if (choice == 0) {
        fetchPc += kInstr;
        perf[P_INSTR_ISSUED]++;
        perf[P_DRAM_RD] += kInstr;
        if (++issued > kMaxInstr) bad("instruction limit exceeded (runaway program?)");
        const uint8_t op = next[0] & 0xFF, ss = (next[0] >> 24) & 0xFF;
        if (op == OP_HALT) {
          halted = true;
        } else if (op == OP_NOP) {
          if (ss != kNoSem) sem[ss]++;
        } else {
          queues[engine_of(op)].push_back(next);
        }
      } else {
        const std::array<uint32_t, 16> in = queues[choice].front();
        queues[choice].pop_front();
        execute(in.data());
        const uint8_t ss = (in[0] >> 24) & 0xFF;
        if (ss != kNoSem) sem[ss]++;
      }
    }
    flush();
    rq_unchecked = true;
    requant_check();
  }
};

}  // namespace llhip

using llhip::Device;

template <class F>
static int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    return llhip::fail(-EINVAL, "%s", e.what());
  }
}

extern "C" {

llhip_device* llhip_dev_create(uint64_t dram_bytes, int epilogue_fusion) {
  Device* d = new Device();
  if (guarded([&] { d->init(dram_bytes, epilogue_fusion != 0); })) {
    delete d;
    return nullptr;
  }
  return reinterpret_cast<llhip_device*>(d);
}

void llhip_dev_destroy(llhip_device* h) { delete reinterpret_cast<Device*>(h); }

int llhip_dev_dram_write(llhip_device* h, uint64_t addr, const void* src, uint64_t n) {
  if (!h || (n && !src)) return llhip::fail(-EINVAL, "dev_dram_write: null argument");
  return guarded([&] { reinterpret_cast<Device*>(h)->write(addr, src, n); });
}

int llhip_dev_dram_read(llhip_device* h, uint64_t addr, void* dst, uint64_t n) {
  if (!h || (n && !dst)) return llhip::fail(-EINVAL, "dev_dram_read: null argument");
  return guarded([&] { reinterpret_cast<Device*>(h)->read(addr, dst, n); });
}

uint64_t llhip_dev_dram_size(const llhip_device* h) { return h ? reinterpret_cast<const Device*>(h)->size : 0; }

int llhip_dev_run(llhip_device* h, uint32_t pc, uint32_t pos, uint64_t* perf) {
  if (!h) return llhip::fail(-EINVAL, "dev_run: null device");
  Device* d = reinterpret_cast<Device*>(h);
  const int rc = guarded([&] { d->run(pc, pos); });
  if (rc) (void)hipStreamSynchronize(d->stream);
  if (!rc && perf) std::memcpy(perf, d->perf, sizeof d->perf);
  return rc;
}

int llhip_dev_sram_snapshot(llhip_device* h, void* dst) {
  if (!h || !dst) return llhip::fail(-EINVAL, "dev_sram_snapshot: null argument");
  Device* d = reinterpret_cast<Device*>(h);
  return guarded([&] {
    llhip::hip_ok(hipMemcpyAsync(dst, d->sram, llhip::kSram, hipMemcpyDeviceToHost, d->stream), "hipMemcpyAsync");
    llhip::hip_ok(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
  });
}

uint32_t llhip_dev_max_attention_head_dim(void) { return 256; }

int llhip_dev_set_interleave(llhip_device* h, uint32_t seed) {
  if (!h) return llhip::fail(-EINVAL, "dev_set_interleave: null device");
  reinterpret_cast<Device*>(h)->seed = seed;
  return 0;
}

void* llhip_dev_dram_ptr(llhip_device* h) { return h ? reinterpret_cast<Device*>(h)->dram : nullptr; }

}  // extern "C"
