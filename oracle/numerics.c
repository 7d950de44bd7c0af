/* CPU oracle, C restatement of the reference's integer datapath.
 *
 * TEST INFRASTRUCTURE ONLY: built into oracle/liboracle.so and loaded by
 * oracle/golden_np.py for large configurations; never linked into the product.
 *
 * Semantics follow python/llaccel/golden.py (cited as golden.py:<line>) and
 * docs/NUMERICS.md of the reference.  Every value is carried in int64 and
 * every product wraps modulo 2^64, which is what the reference's int64 numpy
 * arithmetic does.  Integer sums are exact, so the OpenMP split over rows and
 * columns cannot change a result.
 *
 * The LUTs are handed in by oracle/golden_np.py (orc_set_luts) so that the C and
 * numpy restatements read the same tables; those tables are pinned separately
 * against the constants the reference commits in include/llaccel/luts.h.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int64_t g_sig[257], g_expi[16], g_expf[256];

int orc_set_luts(const uint16_t *sig, const uint16_t *expi, const uint16_t *expf) {
  for (int i = 0; i < 257; ++i) g_sig[i] = sig[i];
  for (int i = 0; i < 16; ++i) g_expi[i] = expi[i];
  for (int i = 0; i < 256; ++i) g_expf[i] = expf[i];
  return 0;
}

int orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

/* wrapping int64 product, as numpy's int64 multiply */
static inline int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }

/* golden.py:35-45 -- round half up: s == 0 -> v, else (v >> s) + bit (s-1) of v */
static inline int64_t rshr(int64_t v, int64_t s) {
  if (s == 0) return v;
  return (v >> s) + ((v >> (s - 1)) & 1);
}
static inline int64_t clamp(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline int64_t sat8(int64_t v) { return clamp(v, -128, 127); }
static inline int64_t sat16(int64_t v) { return clamp(v, -32768, 32767); }
/* golden.py:64-65 */
static inline int64_t mulshift(int64_t v, int64_t M, int64_t S) { return rshr(wmul(v, M), S); }

/* golden.py:68-81: restoring square root, two bits per step */
static int64_t isqrt48(uint64_t t) {
  uint64_t rem = 0, root = 0;
  for (int step = 23; step >= 0; --step) {
    rem = (rem << 2) | ((t >> (2 * step)) & 3u);
    uint64_t cand = (root << 2) | 1u;
    root <<= 1;
    if (cand <= rem) {
      rem -= cand;
      root |= 1u;
    }
  }
  return (int64_t)root;
}

/* golden.py:101-107 */
static inline int64_t silu16(int64_t x, int64_t Mi, int64_t Si, int64_t sh) {
  int64_t u = sat16(mulshift(x, Mi, Si));
  int64_t j = (u >> 8) + 128;
  int64_t f = u & 255;
  int64_t sg = g_sig[j] + (((g_sig[j + 1] - g_sig[j]) * f) >> 8);
  return sat16(rshr(wmul(x, sg), sh));
}

/* exported primitive twins (for the oracle's own cross-checks) */
int64_t orc_rshr(int64_t v, int64_t s) { return rshr(v, s); }
int64_t orc_mulshift(int64_t v, int64_t M, int64_t S) { return mulshift(v, M, S); }
int64_t orc_isqrt48(uint64_t t) { return isqrt48(t); }
int64_t orc_silu16(int64_t x, int64_t Mi, int64_t Si, int64_t sh) { return silu16(x, Mi, Si, sh); }

/* golden.py:124-132, one row; returns -1 when isqrt48's domain is exceeded */
int orc_rmsnorm_row(const int64_t *x, const int64_t *g, int64_t K, int64_t eps_t, int64_t C, int64_t sh_post,
                    int64_t *y) {
  uint64_t ss = 0;
  for (int64_t k = 0; k < K; ++k) ss += (uint64_t)wmul(x[k], x[k]);
  uint64_t tt = ss + (uint64_t)eps_t;
  if (tt >= (1ull << 48)) return -1;
  int64_t r = isqrt48(tt);
  int64_t d = r > 1 ? r : 1;
  int64_t inv = (int64_t)(((uint64_t)C / (uint64_t)d) & 0xFFFFFFFFull);
  if (inv > 65535) inv = 65535;
  for (int64_t k = 0; k < K; ++k) y[k] = sat16(rshr(wmul(wmul(x[k], g[k]), inv), sh_post));
  return 0;
}

/* golden.py:141-152, one row of H heads */
void orc_rope_row(const int64_t *x, int64_t H, int64_t D, const int64_t *c, const int64_t *s, int64_t *y) {
  int64_t half = D / 2;
  for (int64_t h = 0; h < H; ++h)
    for (int64_t i = 0; i < half; ++i) {
      int64_t a = x[h * D + i], b = x[h * D + half + i];
      y[h * D + i] = sat16(rshr(wmul(a, c[i]) - wmul(b, s[i]), 14));
      y[h * D + half + i] = sat16(rshr(wmul(b, c[i]) + wmul(a, s[i]), 14));
    }
}

/* golden.py:162-180 for one (row, head): q[D], keys/vals [T][D] with row stride ld. */
static void attention_head(const int8_t *q, const int8_t *keys, const int8_t *vals, int64_t T, int64_t D, int64_t ld,
                           int64_t Ms, int64_t Ss, int64_t Mo, int64_t So, int64_t pb, int64_t *scores,
                           int64_t *probs, int64_t *acc, int64_t *out) {
  int64_t mx = INT64_MIN;
  for (int64_t t = 0; t < T; ++t) {
    int64_t s = 0;
    const int8_t *k = keys + t * ld;
    for (int64_t d = 0; d < D; ++d) s += (int64_t)q[d] * (int64_t)k[d];
    scores[t] = s;
    if (s > mx) mx = s;
  }
  int64_t total = 0;
  for (int64_t t = 0; t < T; ++t) {
    int64_t z = mulshift(mx - scores[t], Ms, Ss);
    int64_t p = 0;
    if (z < 4096) {
      int64_t zc = z;  /* z >= 0 for valid multipliers; numpy clips the index with min(z, 4095) */
      p = (g_expi[zc >> 8] * g_expf[zc & 255] + (1 << 15)) >> 16;
    }
    probs[t] = p;
    total += p;
  }
  int64_t inv = (int64_t)(((uint64_t)1 << 31) / (uint64_t)(total > 1 ? total : 1) & 0xFFFFFFFFull);
  int64_t cap = ((int64_t)1 << pb) - 1;
  for (int64_t d = 0; d < D; ++d) acc[d] = 0;
  for (int64_t t = 0; t < T; ++t) {
    int64_t pn = rshr(wmul(probs[t], inv), 31 - pb);
    if (pn > cap) pn = cap;
    const int8_t *v = vals + t * ld;
    for (int64_t d = 0; d < D; ++d) acc[d] += pn * (int64_t)v[d];
  }
  for (int64_t d = 0; d < D; ++d) {
    int64_t o = acc[d];
    if (pb == 15) o = rshr(o, 7);
    out[d] = sat8(mulshift(o, Mo, So));
  }
}

int orc_attention_head(const int8_t *q, const int8_t *keys, const int8_t *vals, int64_t T, int64_t D, int64_t Ms,
                       int64_t Ss, int64_t Mo, int64_t So, int64_t pb, int64_t *out) {
  if (pb != 8 && pb != 15) return -1;
  int64_t *work = (int64_t *)malloc(sizeof(int64_t) * (2 * (size_t)T + (size_t)D));
  if (!work) return -2;
  attention_head(q, keys, vals, T, D, D, Ms, Ss, Mo, So, pb, work, work + T, work + 2 * T, out);
  free(work);
  return 0;
}

/* golden.py:353-366: q [M][H*D] i8, caches [Hkv][max_seq][D] i8, out [M][H*D] */
int orc_attention(const int8_t *q, int64_t M, int64_t H, int64_t Hkv, int64_t D, int64_t pos, const int8_t *kc,
                  const int8_t *vc, int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So, int64_t pb,
                  int64_t *out) {
  if (pb != 8 && pb != 15) return -1;
  if (Hkv <= 0 || H % Hkv) return -2;
  int64_t group = H / Hkv;
  int err = 0;
#pragma omp parallel
  {
    int64_t *work = (int64_t *)malloc(sizeof(int64_t) * (2 * (size_t)max_seq + (size_t)D));
    if (!work) {
#pragma omp atomic write
      err = -3;
    } else {
#pragma omp for collapse(2) schedule(dynamic)
      for (int64_t m = 0; m < M; ++m)
        for (int64_t h = 0; h < H; ++h) {
          int64_t T = pos + m + 1;
          int64_t g = h / group;
          attention_head(q + m * H * D + h * D, kc + g * max_seq * D, vc + g * max_seq * D, T, D, D, Ms, Ss, Mo, So,
                         pb, work, work + max_seq, work + 2 * max_seq, out + m * H * D + h * D);
        }
      free(work);
    }
  }
  return err;
}

/* golden.py:316-342.  A i8 [M][K], W i8 [N][K]; epilogue 0 none, 1 resadd, 2 silu, 3 mul. */
int orc_linear(const int8_t *a, int64_t M, int64_t K, const int8_t *w, int64_t N, const int32_t *rq,
               const int32_t *bias, int64_t out_i8, const int16_t *aux, int64_t aux_shift, int64_t epilogue,
               int64_t Mi, int64_t Si, int64_t sh_out, int64_t *out) {
  if (out_i8 && epilogue != 0) return -1;
  if ((epilogue == 1 || epilogue == 3) && !aux) return -2;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t m = 0; m < M; ++m) {
      const int8_t *ar = a + m * K, *wr = w + n * K;
      int64_t acc = 0;
      for (int64_t k0 = 0; k0 < K; k0 += 32768) {
        int64_t k1 = k0 + 32768 < K ? k0 + 32768 : K;
        int32_t part = 0;
        for (int64_t k = k0; k < k1; ++k) part += (int32_t)ar[k] * (int32_t)wr[k];
        acc += part;
      }
      if (bias) acc += bias[n];
      int64_t Mn = rq[2 * n], Sn = rq[2 * n + 1];
      int64_t r = mulshift(acc, Mn, Sn);
      int64_t y;
      if (out_i8) {
        y = sat8(r);
      } else {
        int64_t t = sat16(r);
        switch (epilogue) {
          case 1: y = sat16(t + aux[m * N + n]); break;
          case 2: y = silu16(t, Mi, Si, sh_out); break;
          case 3: y = sat16(rshr(wmul(t, aux[m * N + n]), aux_shift)); break;
          default: y = t;
        }
      }
      out[m * N + n] = y;
    }
  return 0;
}
