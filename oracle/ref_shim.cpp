// extern "C" access to the reference's own header-only C++ numerics
// (include/llaccel/numerics.h + luts.h of /root/reference), compiled in place by
// oracle/Makefile into oracle/_ref/libllaccel_ref.so.  TEST INFRASTRUCTURE ONLY:
// it is used to pin the oracle's primitives against the reference, never by the
// product.  No reference source is copied here; this file only forwards calls.
#include <cstdint>
#include <span>
#include <vector>

#include "llaccel/numerics.h"

namespace n = llaccel::num;

extern "C" {
int64_t ref_rshr(int64_t v, uint32_t s) { return n::rshr(v, s); }
int64_t ref_mulshift(int64_t v, uint32_t M, uint32_t S) { return n::mulshift(v, M, S); }
uint32_t ref_isqrt48(uint64_t t) { return n::isqrt48(t); }
uint32_t ref_udiv(uint64_t a, uint64_t b) { return n::udiv(a, b); }
int64_t ref_requant16(int32_t acc, int32_t M, int32_t S) { return n::requant16(acc, n::RqEntry{M, S}); }
int64_t ref_requant8(int32_t acc, int32_t M, int32_t S) { return n::requant8(acc, n::RqEntry{M, S}); }
int64_t ref_silu16(int64_t x, uint32_t Mi, uint32_t Si, uint32_t sh) { return n::silu16(x, Mi, Si, sh); }
int64_t ref_vmul(int64_t a, int64_t b, uint32_t sh) { return n::vmul(a, b, sh); }
int64_t ref_vadd(int64_t a, int64_t b, uint32_t sh) { return n::vadd(a, b, sh); }
int64_t ref_vquant(int64_t x, uint32_t M, uint32_t S) { return n::vquant(x, M, S); }

void ref_rmsnorm(const int16_t* x, const int16_t* g, int16_t* y, uint32_t K, uint32_t eps_t, uint32_t C,
                 uint32_t sh_post) {
  n::rmsnorm(std::span<const int16_t>(x, K), std::span<const int16_t>(g, K), std::span<int16_t>(y, K), eps_t, C,
             sh_post);
}

void ref_rope(const int16_t* x, int16_t* y, uint32_t H, uint32_t D, const int16_t* c, const int16_t* s) {
  n::rope(std::span<const int16_t>(x, size_t(H) * D), std::span<int16_t>(y, size_t(H) * D), H, D,
          std::span<const int16_t>(c, D / 2), std::span<const int16_t>(s, D / 2));
}

// keys/vals: [T][D] contiguous
void ref_attention_head(const int8_t* q, uint32_t D, uint32_t T, const int8_t* keys, const int8_t* vals, uint32_t Ms,
                        uint32_t Ss, uint32_t Mo, uint32_t So, int8_t* out, int wide) {
  std::vector<int32_t> scores;
  std::vector<uint16_t> probs;
  n::attention_head(
      std::span<const int8_t>(q, D), D, T, [&](uint32_t t) { return keys + size_t(t) * D; },
      [&](uint32_t t) { return vals + size_t(t) * D; }, Ms, Ss, Mo, So, std::span<int8_t>(out, D), scores, probs,
      wide != 0);
}

void ref_luts(uint16_t* sig, uint16_t* expi, uint16_t* expf) {
  for (size_t i = 0; i < n::kSigmoidLut.size(); ++i) sig[i] = n::kSigmoidLut[i];
  for (size_t i = 0; i < n::kExpIntLut.size(); ++i) expi[i] = n::kExpIntLut[i];
  for (size_t i = 0; i < n::kExpFracLut.size(); ++i) expf[i] = n::kExpFracLut[i];
}
}
