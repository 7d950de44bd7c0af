// C-ABI core of libllhip: error state, LUT constants, workspace size and the
// elementwise int64 primitives of golden.py:35-120.
#include <cstdarg>
#include <cstring>

#include "../../include/llhip.h"
#include "common.h"

namespace llhip {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int current_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// ---------------------------------------------------------------------------------------
// elementwise int64 primitives
// ---------------------------------------------------------------------------------------
enum PrimOp : int {
  P_RSHR = 0,
  P_SAT8,
  P_SATU8,
  P_SAT16,
  P_SATU16,
  P_MULSHIFT,
  P_REQUANT16,
  P_REQUANT8,
  P_ISQRT48,
  P_UDIV,
  P_SILU16,
  P_VMUL,
  P_VADD,
  P_VQUANT,
};

struct PrimArgs {
  const int64_t* a;
  const int64_t* b;
  const int64_t* c;
  int64_t s0, s1, s2;  // scalar parameters
  int64_t n;
  int64_t* out;
  int op;
};

__global__ void prim_kernel(PrimArgs p) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < p.n; i += stride) {
    int64_t a = p.a[i];
    int64_t r;
    switch (p.op) {
      case P_RSHR: r = rshr(a, (int)p.b[i]); break;
      case P_SAT8: r = sat8(a); break;
      case P_SATU8: r = clamp64(a, 0, 255); break;
      case P_SAT16: r = sat16(a); break;
      case P_SATU16: r = clamp64(a, 0, 65535); break;
      case P_MULSHIFT: r = mulshift(a, p.b[i], (int)p.c[i]); break;
      case P_REQUANT16: r = sat16(mulshift(a, p.b[i], (int)p.c[i])); break;
      case P_REQUANT8: r = sat8(mulshift(a, p.b[i], (int)p.c[i])); break;
      case P_ISQRT48: r = isqrt48((uint64_t)a); break;
      case P_UDIV: {
        uint64_t d = p.b[i] > 1 ? (uint64_t)p.b[i] : 1u;
        r = (int64_t)(((uint64_t)a / d) & 0xFFFFFFFFull);
        break;
      }
      case P_SILU16: r = silu16(a, p.s0, (int)p.s1, (int)p.s2); break;
      case P_VMUL: r = sat16(rshr(wmul(a, p.b[i]), (int)p.s0)); break;
      case P_VADD: r = sat16(a + rshr(p.b[i], (int)p.s0)); break;
      case P_VQUANT: r = sat8(mulshift(a, p.s0, (int)p.s1)); break;
      default: r = 0;
    }
    p.out[i] = r;
  }
}

static int launch_prim(PrimArgs p, void* stream) {
  if (p.n < 0) return fail(-EINVAL, "negative element count");
  if (p.n == 0) return 0;
  int64_t blocks = ceil_div(p.n, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(prim_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  LLHIP_LAUNCH_CHECK();
  return 0;
}

}  // namespace llhip

using namespace llhip;

extern "C" {

int llhip_abi_version(void) { return LLHIP_ABI_VERSION; }

const char* llhip_last_error(void) { return g_last_error.c_str(); }

// split-K GEMM partials (16 rows x 32768 columns of int32) + per-tile arrival counters,
// attention partials; see gemm.hip / attn.hip
int64_t llhip_workspace_bytes(void) { return (int64_t)32 << 20; }

int llhip_rshr(const int64_t* v, const int64_t* s, int64_t n, int64_t* out, void* stream) {
  return launch_prim(PrimArgs{v, s, nullptr, 0, 0, 0, n, out, P_RSHR}, stream);
}

int llhip_sat(const int64_t* v, int64_t n, int kind, int64_t* out, void* stream) {
  if (kind < 0 || kind > 3) return fail(-EINVAL, "sat kind %d", kind);
  return launch_prim(PrimArgs{v, nullptr, nullptr, 0, 0, 0, n, out, P_SAT8 + kind}, stream);
}

int llhip_mulshift(const int64_t* v, const int64_t* M, const int64_t* S, int64_t n, int64_t* out, void* stream) {
  return launch_prim(PrimArgs{v, M, S, 0, 0, 0, n, out, P_MULSHIFT}, stream);
}

int llhip_requant(const int64_t* acc, const int64_t* M, const int64_t* S, int64_t n, int bits, int64_t* out,
                  void* stream) {
  if (bits != 8 && bits != 16) return fail(-EINVAL, "requant bits %d", bits);
  return launch_prim(PrimArgs{acc, M, S, 0, 0, 0, n, out, bits == 16 ? P_REQUANT16 : P_REQUANT8}, stream);
}

int llhip_isqrt48(const int64_t* t, int64_t n, int64_t* out, void* stream) {
  return launch_prim(PrimArgs{t, nullptr, nullptr, 0, 0, 0, n, out, P_ISQRT48}, stream);
}

int llhip_udiv(const int64_t* a, const int64_t* b, int64_t n, int64_t* out, void* stream) {
  return launch_prim(PrimArgs{a, b, nullptr, 0, 0, 0, n, out, P_UDIV}, stream);
}

int llhip_silu16_i64(const int64_t* x, int64_t n, int64_t Mi, int64_t Si, int64_t sh_out, int64_t* out,
                     void* stream) {
  if (!shift_ok(Si) || !shift_ok(sh_out)) return fail(-EINVAL, "silu shift out of [0,63]");
  return launch_prim(PrimArgs{x, nullptr, nullptr, Mi, Si, sh_out, n, out, P_SILU16}, stream);
}

int llhip_vmul_i64(const int64_t* a, const int64_t* b, int64_t n, int64_t sh, int64_t* out, void* stream) {
  if (!shift_ok(sh)) return fail(-EINVAL, "vmul shift out of [0,63]");
  return launch_prim(PrimArgs{a, b, nullptr, sh, 0, 0, n, out, P_VMUL}, stream);
}

int llhip_vadd_i64(const int64_t* a, const int64_t* b, int64_t n, int64_t sh_b, int64_t* out, void* stream) {
  if (!shift_ok(sh_b)) return fail(-EINVAL, "vadd shift out of [0,63]");
  return launch_prim(PrimArgs{a, b, nullptr, sh_b, 0, 0, n, out, P_VADD}, stream);
}

int llhip_vquant_i64(const int64_t* x, int64_t n, int64_t M, int64_t S, int64_t* out, void* stream) {
  if (!shift_ok(S)) return fail(-EINVAL, "vquant shift out of [0,63]");
  return launch_prim(PrimArgs{x, nullptr, nullptr, M, S, 0, n, out, P_VQUANT}, stream);
}

}  // extern "C"
