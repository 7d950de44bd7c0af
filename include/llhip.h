/* libllhip -- MI355X (gfx950) kernels of llaccel's bit-exact integer decoder datapath.
 *
 * C ABI loaded with ctypes by llaccel_amd/_lib.py.  The reference has no FFI for this
 * path: its "plugin API" is the Python surface of python/llaccel/golden.py.  Each entry
 * point below replaces the golden.py function cited beside it, computing the same
 * integers on the GPU.
 *
 * Conventions
 *   - Every tensor pointer is a DEVICE pointer; the caller owns all memory.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); work is stream-ordered
 *     and asynchronous.
 *   - Return 0 on success; -EINVAL (-22) for a bad shape or parameter (shift outside
 *     [0,63], multiplier outside u32, ...), -ERANGE (-34) for a position or domain error,
 *     -EIO (-5) for a HIP runtime error.  llhip_last_error() returns the thread's message.
 *   - Positions: functions taking (pos, pos_dev) use *pos_dev when pos_dev is non-NULL
 *     (device-resident decode state, e.g. inside a captured graph), else pos.
 *   - `ws` is a caller-allocated workspace of llhip_workspace_bytes() bytes, zero-filled
 *     once at allocation.  Every call leaves the parts that must start at zero zero-filled
 *     again, so it needs no clearing between calls (and none inside a captured graph).
 *     Calls that share one workspace must be ordered on one stream.  llhip_linear uses it
 *     for split-K partial sums when the output has too few tiles to fill the GPU (a NULL ws
 *     only disables that split).
 */
#ifndef LLHIP_H
#define LLHIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLHIP_ABI_VERSION 2

int llhip_abi_version(void);
const char* llhip_last_error(void);
/* bytes of the shared workspace used by llhip_linear / llhip_attention */
int64_t llhip_workspace_bytes(void);

/* ---- elementwise primitives over n int64 values (operands pre-broadcast by the host) ---- */
/* golden.py:35-45  rshr(v, s), s in [0,63] */
int llhip_rshr(const int64_t* v, const int64_t* s, int64_t n, int64_t* out, void* stream);
/* golden.py:48-61  kind 0 sat8, 1 satu8, 2 sat16, 3 satu16 */
int llhip_sat(const int64_t* v, int64_t n, int kind, int64_t* out, void* stream);
/* golden.py:64-65  mulshift(v, M, S) = rshr(v*M, S), int64 wrapping product */
int llhip_mulshift(const int64_t* v, const int64_t* M, const int64_t* S, int64_t n, int64_t* out, void* stream);
/* golden.py:92-97  requant16 (bits 16) / requant8 (bits 8) */
int llhip_requant(const int64_t* acc, const int64_t* M, const int64_t* S, int64_t n, int bits, int64_t* out,
                  void* stream);
/* golden.py:68-81  isqrt48; each t must be in [0, 2^48) */
int llhip_isqrt48(const int64_t* t, int64_t n, int64_t* out, void* stream);
/* golden.py:84-88  udiv(a, b) = (a // max(b,1)) & 0xFFFFFFFF; a, b >= 0 */
int llhip_udiv(const int64_t* a, const int64_t* b, int64_t n, int64_t* out, void* stream);
/* golden.py:101-107 silu16(x, Mi, Si, sh_out) on int64 values */
int llhip_silu16_i64(const int64_t* x, int64_t n, int64_t Mi, int64_t Si, int64_t sh_out, int64_t* out,
                     void* stream);
/* golden.py:111-112 vmul on int64 values */
int llhip_vmul_i64(const int64_t* a, const int64_t* b, int64_t n, int64_t sh, int64_t* out, void* stream);
/* golden.py:115-116 vadd on int64 values */
int llhip_vadd_i64(const int64_t* a, const int64_t* b, int64_t n, int64_t sh_b, int64_t* out, void* stream);
/* golden.py:119-120 vquant on int64 values */
int llhip_vquant_i64(const int64_t* x, int64_t n, int64_t M, int64_t S, int64_t* out, void* stream);

/* ---- vec engine on datapath types (NUMERICS.md: x, g i16; quant out i8) ---- */
/* golden.py:124-137  RMSNorm of `rows` rows of K i16 values (row strides ldx/ldy elements) */
int llhip_rmsnorm(const int16_t* x, int64_t rows, int64_t K, int64_t ldx, const int16_t* g, int64_t eps_t, int64_t C,
                  int64_t sh_post, int16_t* y, int64_t ldy, void* stream);
/* golden.py:119-120  vquant i16 -> i8 over n values */
int llhip_quant(const int16_t* x, int64_t n, int64_t M, int64_t S, int8_t* y, void* stream);
/* golden.py:101-107  silu16 i16 -> i16 */
int llhip_silu(const int16_t* x, int64_t n, int64_t Mi, int64_t Si, int64_t sh_out, int16_t* y, void* stream);
/* golden.py:111-112  vmul */
int llhip_vmul(const int16_t* a, const int16_t* b, int64_t n, int64_t sh, int16_t* y, void* stream);
/* golden.py:115-116  vadd */
int llhip_vadd(const int16_t* a, const int16_t* b, int64_t n, int64_t sh_b, int16_t* y, void* stream);
/* golden.py:141-158  RoPE of x [M][H*D] (row stride ldx) with Q1.14 tables [max_seq][D/2]; row m at
 * pos+m (pos read from pos_dev when non-NULL), or at row_pos[m] when row_pos (int32 [M], device)
 * is non-NULL (one sequence per row). */
int llhip_rope(const int16_t* x, int64_t M, int64_t H, int64_t D, int64_t ldx, const int16_t* cos_tab,
               const int16_t* sin_tab, int64_t table_rows, int64_t pos, const int32_t* pos_dev,
               const int32_t* row_pos, int16_t* y, int64_t ldy, void* stream);
/* golden.py:141-158 + 119-120 [+ 344-351]  RoPE of M rows of H heads, then quant (qM, qS) of the
 * rotated rows: y i16 and yq i8, both [M][H*D].  With kc non-NULL the quantised rows also go to the
 * K cache at their positions, and with vc non-NULL the v rows [M][ldv] to the V cache (the layer's
 * kv_write; caches [slots][H][max_seq][D], slot m at m * slot_stride with row_pos). */
int llhip_rope_quant(const int16_t* x, int64_t M, int64_t H, int64_t D, int64_t ldx, const int16_t* cos_tab,
                     const int16_t* sin_tab, int64_t table_rows, int64_t pos, const int32_t* pos_dev,
                     const int32_t* row_pos, int16_t* y, int8_t* yq, int64_t qM, int64_t qS, int8_t* kc,
                     const int8_t* v, int64_t ldv, int8_t* vc, int64_t max_seq, int64_t slot_stride, void* stream);
/* the arguments of one llhip_rope_quant call */
typedef struct llhip_rope_quant_desc {
  const void* x;        /* i16 [M][ldx] */
  int64_t M, H, D, ldx;
  const void* cos_tab;  /* i16 [table_rows][D/2] */
  const void* sin_tab;
  int64_t table_rows, pos;
  const void* pos_dev;  /* int32, or NULL: pos */
  const void* row_pos;  /* int32 [M] per-row positions, or NULL */
  void* y;              /* i16 [M][H*D] */
  void* yq;             /* i8 [M][H*D] */
  int64_t qM, qS;
  void* kc;             /* K cache or NULL */
  const void* v;        /* v rows [M][ldv] (with vc) */
  int64_t ldv;
  void* vc;             /* V cache or NULL */
  int64_t max_seq, slot_stride;
  int64_t seq_rows;     /* > 0 (no pos_dev, no row_pos): M / seq_rows sequences of seq_rows rows; row m is
                         * at position pos + m % seq_rows, its caches at kc/vc + (m / seq_rows) * slot_stride
                         * (a batch of prompts prefilled in one launch); 0: off */
} llhip_rope_quant_desc;
/* golden.py:141-158 + 119-120 [+ 344-351]  two llhip_rope_quant calls in one launch (a prompt
 * chunk's query rows, then its key rows with the layer's kv_write): the same checks and results as
 * the two calls in order. */
int llhip_rope_quant2(const llhip_rope_quant_desc* a, const llhip_rope_quant_desc* b, void* stream);

/* ---- gemm engine ---- */
/* golden.py:316-342  out[M][N] = epilogue(requant(A[M][K] . W[N][K]^T + bias)).
 * A i8 (row stride lda), W i8 row-major [N][K], rq int32 pairs [N][2] = {M_n, S_n},
 * bias int32 [N] or NULL, aux i16 [M][N] (row stride ldaux) for resadd/mul.
 * epilogue: 0 none, 1 resadd, 2 silu, 3 mul.  out_i8 selects i8 output (epilogue 0 only),
 * otherwise i16.  The rq table's S_n must lie in [0,63], which the caller checks.  The silu
 * multiplier silu_Mi is u32 and its shifts lie in [0,63], as for llhip_silu. */
int llhip_linear(const int8_t* A, int64_t M, int64_t K, int64_t lda, const int8_t* W, int64_t N, const int32_t* rq,
                 const int32_t* bias, int epilogue, const int16_t* aux, int64_t ldaux, int64_t aux_shift,
                 int64_t silu_Mi, int64_t silu_Si, int64_t silu_sh, int out_i8, void* out, int64_t ldo, void* ws,
                 void* stream);
/* golden.py:316-342 (silu and mul epilogues) + 119-120  the gate and up projections of an MLP over
 * M rows in one launch: sg = silu16(requant16(A . Wg^T + bg)), f = sat16(rshr(requant16(A . Wu^T +
 * bu) * sg, mul_sh)), fq = quant(f), outputs [M][ld] (i16, i16, i8) -- the values of the gate
 * linear, the up linear and the quant run one by one.  sg_out and f_out may be NULL (those rows
 * are then not written) when K % 64 == 0, lda % 16 == 0 and A, Wg, Wu are 16-byte aligned (the
 * one-launch path), and are an error otherwise.  fq_out is always required. */
typedef struct llhip_gate_up_desc {
  const void* A;  /* i8 [M][lda] */
  int64_t M, K, lda;
  const void* Wg; const void* rqg; const void* bg;  /* int8 [N][K], int32 [N][2], int32 [N] or NULL */
  const void* Wu; const void* rqu; const void* bu;
  int64_t N, ld;
  int64_t silu_Mi, silu_Si, silu_sh, mul_sh, fq_M, fq_S;
  void* sg_out; void* f_out; void* fq_out;
} llhip_gate_up_desc;
int llhip_gate_up(const llhip_gate_up_desc* d, void* stream);

/* golden.py:316-342 for several linears of one input in one launch (the q, k, v projections of a
 * prompt chunk): out_q = requant(A . W_q^T + bias_q), epilogue none, i8 or i16 output.  At most 4
 * problems. */
typedef struct llhip_linear_problem {
  const void* W;     /* int8 [N][K] */
  int64_t N;
  const void* rq;    /* int32 [N][2] */
  const void* bias;  /* int32 [N] or NULL */
  void* out;         /* [M][ldo] i8 or i16 */
  int64_t ldo, out_i8;
} llhip_linear_problem;
int llhip_linear_group(const int8_t* A, int64_t M, int64_t K, int64_t lda, int64_t count,
                       const llhip_linear_problem* probs, void* ws, void* stream);
/* golden.py:316-342 + 141-158 + 119-120 + 344-351 -- the q, k, v projections of a prompt chunk
 * (probs[0..2]: q and k with i16 outputs, v with i8 output, N multiples of 64) and the rope -> quant
 * of the query rows (rq) and of the key rows with the K/V cache write (rk, its v = probs[2].out) in
 * ONE launch: llhip_linear_group followed by llhip_rope_quant2 with x = the q and k outputs, every
 * output of both written.  head_dim 64, K a multiple of 128, 16-byte aligned rows, tables and
 * caches, slot_stride a multiple of 16.  rq and rk give the same positions and tables. */
int llhip_linear_group_rope(const int8_t* A, int64_t M, int64_t K, int64_t lda, const llhip_linear_problem* probs,
                            const llhip_rope_quant_desc* rq, const llhip_rope_quant_desc* rk, void* ws,
                            void* stream);

/* golden.py:217-240  exact integer A[M][K] (int64) . W[N][K]^T (int8) -> int64 [M][N] */
int llhip_exact_matmul(const int64_t* A, int64_t M, int64_t K, const int8_t* W, int64_t N, int64_t* out,
                       void* stream);

/* ---- attn engine ---- */
/* Batch decode (row_pos non-NULL, int32 [M] on the device): row m is its own sequence at position
 * row_pos[m], with its caches at kc/vc + m * slot_stride (slot_stride >= Hkv * max_seq * D).
 * Otherwise row m sits at pos + m (pos read from pos_dev when non-NULL) in the caches at kc/vc. */
/* golden.py:344-351  K/V rows of M positions into caches [Hkv][max_seq][D] at pos+m */
int llhip_kv_write(const int8_t* k, const int8_t* v, int64_t M, int64_t Hkv, int64_t D, int64_t ldk, int64_t ldv,
                   int64_t pos, const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, int8_t* kc,
                   int8_t* vc, int64_t max_seq, void* stream);
/* golden.py:353-366 (+ attention_head golden.py:162-180)  causal GQA attention of q [M][H*D]
 * over caches [Hkv][max_seq][D]; row m sees keys 0..pos+m.  prob_bits 8 or 15. */
int llhip_attention(const int8_t* q, int64_t M, int64_t H, int64_t Hkv, int64_t D, int64_t ldq, int64_t pos,
                    const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, const int8_t* kc,
                    const int8_t* vc, int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So,
                    int64_t prob_bits, int8_t* out, int64_t ldo, void* ws, void* stream);

/* golden.py:353-366 for a batch of prompts prefilled in one launch (golden.py:379-390 per prompt):
 * M / seq_rows sequences of seq_rows rows, seq_rows a multiple of 16.  Row m is row m % seq_rows of
 * sequence m / seq_rows, at position pos + m % seq_rows, over the caches at kc/vc + (m / seq_rows) *
 * slot_stride, slot_stride >= Hkv * max_seq * D.  A row sees the keys of its own sequence up to its
 * position: the same results per sequence as llhip_attention on that sequence's rows alone. */
int llhip_attention_seqs(const int8_t* q, int64_t M, int64_t seq_rows, int64_t H, int64_t Hkv, int64_t D,
                         int64_t ldq, int64_t pos, const int8_t* kc, const int8_t* vc, int64_t slot_stride,
                         int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So, int64_t prob_bits,
                         int8_t* out, int64_t ldo, void* stream);

/* No counterpart in the reference: llhip_attention for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, results and errors as llhip_attention without `ws`: the split-context partials of
 * long contexts live in a static device array of LLHIP_ATTENTION_NOALLOC_SCRATCH bytes per GPU,
 * held until the process ends.  A launch plan whose partials would not fit takes fewer key splits
 * (or none), so every input llhip_attention accepts is accepted; the plan's size is checked before
 * any launch.  The call allocates nothing (no hipMalloc/hipFree).  Every call on one GPU shares
 * that GPU's array, and the partials are written in full before they are read within a call, so
 * nothing carries over between calls -- but calls that overlap on one GPU (other streams, other
 * threads) race on it. */
#define LLHIP_ATTENTION_NOALLOC_SCRATCH (4 << 20)
int llhip_attention_noalloc(const int8_t* q, int64_t M, int64_t H, int64_t Hkv, int64_t D, int64_t ldq, int64_t pos,
                            const int32_t* pos_dev, const int32_t* row_pos, int64_t slot_stride, const int8_t* kc,
                            const int8_t* vc, int64_t max_seq, int64_t Ms, int64_t Ss, int64_t Mo, int64_t So,
                            int64_t prob_bits, int8_t* out, int64_t ldo, void* stream);

/* ---- host-loop helpers ---- */
/* golden.py:369-373  rows[m] = embed[tokens[m]] for m < n_tokens, zero for n_tokens <= m < M.
 * tokens are int32 row indices already resolved by the caller to [0, vocab_rows). */
int llhip_embed_rows(const int16_t* embed, int64_t vocab_rows, int64_t dim, const int32_t* tokens, int64_t n_tokens,
                     int64_t M, int16_t* rows, void* stream);
/* golden.py:376-377  idx[r] = first argmax of logits[r][0:vocab] (row stride ld) */
int llhip_argmax_i16(const int16_t* logits, int64_t rows, int64_t ld, int64_t vocab, int32_t* idx, void* stream);

/* golden.py:376-377 + the launch record of golden.py:411-414, in decode-loop form: first argmax
 * of logits[0:vocab] -> *token; when *step < ring_cap the row is copied to ring_rows[*step]
 * (row stride ring_ld) and the token to ring_tokens[*step]; then *pos += 1 and *step += 1.
 * Everything stays on the device, so a captured decode launch needs no host round trip. */
int llhip_greedy_step(const int16_t* logits, int64_t vocab, int32_t* token, int32_t* pos, int32_t* step,
                      int16_t* ring_rows, int64_t ring_ld, int32_t* ring_tokens, int64_t ring_cap, void* ws,
                      void* stream);

/* golden.py:376-377 + the launch record of golden.py:411-414 for a batch decode launch, one
 * sequence per row: tokens[r] = first argmax of logits[r][0:vocab], rows ld elements apart.  With
 * s = positions[r] - base[r], when 0 <= s < ring_cap the row goes to ring_rows[s][r] (rows of
 * ring_ld elements, [ring_cap][rows] of them) and the token to ring_tokens[s][r]; then
 * positions[r] += 1. */
int llhip_greedy_rows(const int16_t* logits, int64_t rows, int64_t ld, int64_t vocab, int32_t* tokens,
                      int32_t* positions, const int32_t* base, int16_t* ring_rows, int64_t ring_ld,
                      int32_t* ring_tokens, int64_t ring_cap, void* stream);

/* ---- record verification on the device (a long run checked without downloading its rows) ---- */
/* verify.py:80-104 (compare_sim: records equal element by element) on device-resident i16 rows:
 * *out = smallest flat index r * cols + c with a[r][c] != b[r][c], or -1 when the row sets are
 * equal (out is an int64 in device memory) */
int llhip_rows_first_mismatch_i16(const int16_t* a, int64_t lda, const int16_t* b, int64_t ldb, int64_t rows,
                                  int64_t cols, int64_t* out, void* stream);
/* verify.py:80-104 by checksum: out[r] = sum_c (c + 1) * (uint16)x[r][c] modulo 2^64, so two runs
 * are compared by rows * 8 bytes (llaccel_amd/verify.py computes the same on the host) */
int llhip_rows_checksum_i16(const int16_t* x, int64_t ld, int64_t rows, int64_t cols, uint64_t* out, void* stream);

/* ---- quantizer (the float -> integer conversions of the qgraph producer) ----
 * refquant.py:137-141 + 119-125  per-output-channel int8 weights of w f32 [N][K] (row stride ldw):
 * scales[n] = max|w[n,:]| / 127 as a double (1 for an all-zero row), q[n][k] = llround(clip(w[n][k] /
 * scales[n], -128, 127)), llround rounding halves away from zero (refquant.py:61-72).  A non-finite
 * weight sets *status to 1 (status is an int32 in device memory, zeroed by the caller). */
int llhip_quant_rows_i8(const float* w, int64_t N, int64_t K, int64_t ldw, int8_t* q, int64_t ldq, double* scales,
                        int32_t* status, void* stream);
/* refquant.py:128-134  i16 tensor at exponent e: y = llround(clip(x * 2^-e, -32768, 32767)). */
int llhip_quant_i16(const float* x, int64_t n, int64_t e, int16_t* y, int32_t* status, void* stream);

/* ---- fused decoder blocks (M <= 16 rows per launch) ----
 * Each computes a run of consecutive qgraph ops in one launch and writes every activation
 * those ops name, with the values the separate entry points above produce.  Row strides of
 * the i16 rows are ldx elements; i8 rows are K (or N) elements.  K % 8 == 0. */
typedef struct llhip_norm_quant_desc {
  const void* x;     /* i16 [M][ldx] input rows */
  const void* gamma; /* i16 [K] */
  void* h_out;       /* i16 [M][ldx] normalised rows, or NULL */
  void* hq_out;      /* i8 [M][K] quantised rows, or NULL */
  int64_t ldx, K, eps_t, C, sh_post, Mq, Sq;
  int64_t prequant;  /* fused kernels: nonzero when h_out/hq_out already hold the rows (written by
                      * llhip_rmsnorm_quant); the kernel then reads hq_out instead of normalising x */
} llhip_norm_quant_desc;

/* golden.py:124-137 + 119-120  rmsnorm then quant of M rows in one launch (one workgroup per row):
 * h_out = rmsnorm(x), hq_out = quant(h_out).  Multi-row fused launches run it first (prequant). */
int llhip_rmsnorm_quant(const llhip_norm_quant_desc* d, int64_t M, void* stream);
/* golden.py:316-342 (resadd epilogue) + 124-137 + 119-120  llhip_linear with the resadd epilogue
 * (out i16 [M][ldo]) followed by llhip_rmsnorm_quant(norm, M) of its output rows (norm->x == out,
 * norm->ldx == ldo, norm->K == N): the same results; a launch split along K finishes its partial
 * sums and normalises the rows in one kernel. */
int llhip_linear_norm(const int8_t* A, int64_t M, int64_t K, int64_t lda, const int8_t* W, int64_t N, const int32_t* rq,
                      const int32_t* bias, const int16_t* aux, int64_t ldaux, int16_t* out, int64_t ldo,
                      const llhip_norm_quant_desc* norm, void* ws, void* stream);

typedef struct llhip_attn_in_desc {
  llhip_norm_quant_desc pre;
  const void* W[3];    /* q, k, v weights i8 [N][K] */
  const void* rq[3];   /* int32 [N][2] */
  const void* bias[3]; /* int32 [N] or NULL */
  void* lin_out[3];    /* q i16 [M][H*D], k i16 [M][Hkv*D], v i8 [M][Hkv*D] */
  const void* nrm_gamma[2]; /* Q/K RMSNorm gamma i16 [D] (has_norm) */
  void* nrm_out[2];
  int64_t nrm_eps[2], nrm_C[2], nrm_sh[2];
  const void* cos_tab; /* i16 [max_seq][D/2] */
  const void* sin_tab;
  const void* pos_dev; /* int32 device position or NULL */
  void* rope_out[2];   /* i16 rows */
  void* quant_out[2];  /* i8 rows */
  int64_t quant_M[2], quant_S[2];
  void* kc; /* int8 caches [Hkv][max_seq][D] */
  void* vc;
  int64_t max_seq, M, H, Hkv, D, pos, has_norm;
  const void* row_pos; /* int32 [M] device positions, one sequence per row (batch decode), or NULL */
  int64_t slot_stride; /* with row_pos: elements between the caches of rows m and m + 1 */
} llhip_attn_in_desc;

/* golden.py:286-300 -- rmsnorm, quant, linear q/k/v (+bias), [rmsnorm heads q/k], rope q/k,
 * quant q/k, kv_write: one workgroup per head block. */
int llhip_attn_in(const llhip_attn_in_desc* d, void* stream);

typedef struct llhip_mlp_in_desc {
  llhip_norm_quant_desc pre;
  const void* Wg; const void* Wu;   /* i8 [N][K] */
  const void* rqg; const void* rqu; /* int32 [N][2] */
  const void* bg; const void* bu;   /* int32 [N] or NULL */
  void* g_out; void* u_out;         /* i16 [M][N] (unfused graphs) or NULL */
  void* sg_out; void* f_out;        /* i16 [M][N] */
  void* fq_out;                     /* i8 [M][N] */
  int64_t silu_Mi, silu_Si, silu_sh, mul_sh, fq_M, fq_S, M, N;
} llhip_mlp_in_desc;

/* golden.py:286-309 + 332-342 -- rmsnorm, quant, linear gate (silu epilogue) and up (mul
 * epilogue) [or linear g, linear u, silu, mul], quant. */
int llhip_mlp_in(const llhip_mlp_in_desc* d, void* stream);

typedef struct llhip_norm_linear_desc {
  llhip_norm_quant_desc pre;
  const void* W; const void* rq; const void* bias; const void* aux;
  void* out; /* [M][N] i16 or i8 */
  int64_t epilogue, aux_shift, silu_Mi, silu_Si, silu_sh, out_i8, M, N;
} llhip_norm_linear_desc;

/* golden.py:286-296 + 316-342 -- rmsnorm, quant, one linear with any epilogue. */
int llhip_norm_linear(const llhip_norm_linear_desc* d, void* stream);

/* ---- decode chain: one decode row of a fused graph in three launches per layer ----
 * A decode launch (M = 1) of the reference's fused qgraph (golden.py:275-314) runs each layer as
 *   llhip_dec_attn_in   : [finish the previous layer's down projection] rmsnorm, quant, q/k/v, rope,
 *                         quant, kv_write, as the attn_in run above;
 *   llhip_dec_attention : attention, then the output projection's partial sums per head;
 *   llhip_dec_mlp       : finish the output projection, rmsnorm, quant, gate/up, quant, then the down
 *                         projection's partial sums per 16 FFN columns;
 * and the final norm + lm_head + greedy step as llhip_dec_finish + llhip_dec_head + llhip_dec_greedy.  The output (wo)
 * and down (wd) projections -- linear with the resadd epilogue, golden.py:316-342 -- are computed as
 * exact int32 partial sums of disjoint K ranges added into accumulator rows with atomics; the next
 * launch finishes them (bias, requant16, resadd) in its prologue.  Integer addition is associative,
 * so every activation equals the separate linear's.  Every activation the ops name is written. */
typedef struct llhip_resid_desc {
  const void* acc;  /* int32 [R][N] partial sums of the projection; NULL: the row is pre.x itself */
  int64_t R;        /* accumulator rows (1..8) whose sum is the projection */
  const void* rq;   /* int32 [N][2] the projection's requant pairs */
  const void* bias; /* int32 [N] or NULL */
  const void* aux;  /* i16 [N] the residual of the resadd epilogue */
  void* x_out;      /* i16 [N] the finished row (the projection's output activation) */
} llhip_resid_desc;

/* golden.py:286-300 + 316-342 -- llhip_attn_in for one row whose input row is the resadd output of
 * the previous projection when r->acc is non-NULL (written to r->x_out), else pre.x; it also clears
 * zero[0..zero_n) (int32, 16-byte aligned) for the attention's output projection. */
int llhip_dec_attn_in(const llhip_attn_in_desc* d, const llhip_resid_desc* r, void* zero, int64_t zero_n,
                      void* stream);

typedef struct llhip_dec_attn_desc {
  const void* q;        /* i8 [H*D] */
  const void* kc;       /* int8 caches [Hkv][max_seq][D] */
  const void* vc;
  void* out;            /* i8 [H*D] the attention activation */
  const void* pos_dev;  /* int32 device position, or NULL: pos */
  int64_t pos, H, Hkv, D, max_seq, Ms, Ss, Mo, So, prob_bits;
  const void* wo_panel; /* i8 [H][N][D]: the output projection W[n][h*D + d] at [h][n][d] */
  int64_t N;            /* the output projection's width */
  void* acc;            /* int32 [N], zero on entry: receives the H per-head partial sums */
  void* zero;           /* int32 [zero_n] cleared for the down projection (16-byte aligned) */
  int64_t zero_n;
  void* state;          /* or NULL: zero-filled device memory owned by the caller, kept across launches,
                         * of the size llhip_dec_attn_state_bytes gives; long contexts then run as ONE
                         * launch whose H x S workgroups exchange their partials through it */
  int64_t state_bytes;
} llhip_dec_attn_desc;

/* golden.py:353-366 + 316-342 -- causal GQA attention of one row, then each head's partial sums of
 * the output projection (K range h*D..h*D+D-1) added into acc.  ws as for llhip_attention.  With
 * `state`, a long context (>= 2048 keys, head_dim 64 or 128) is one launch of H x S workgroups (S
 * <= 16 splits of the keys per head) that wait for each other with bounded waits; a timed-out wait
 * sets the state's error word (read with llhip_dec_attn_status), and later launches with that state
 * do nothing. */
int llhip_dec_attention(const llhip_dec_attn_desc* d, void* ws, void* stream);
/* golden.py:353-366 -- bytes of the state of llhip_dec_attention's one-launch form for H heads of
 * head_dim D (at most 16 splits per head). */
int64_t llhip_dec_attn_state_bytes(int64_t H, int64_t D);
/* golden.py:353-366 -- synchronous: *launches = one-launch attentions completed with this state,
 * *err = nonzero when one hit a bounded-wait timeout (sticky). */
int llhip_dec_attn_status(const void* state, int64_t* launches, int64_t* err);

/* golden.py:286-309 + 316-342 -- llhip_mlp_in for one row whose input is the resadd output of the
 * output projection (r), then the down projection's partial sums of each workgroup's 16 FFN columns
 * added into wd_acc [R][N_out] (zero on entry; workgroup b adds into row b % R).  wd_panel is i8
 * [ceil(N/16)][N_out][16]: W_down[n][16b + j] at [b][n][j], zero bytes for 16b + j >= N. */
int llhip_dec_mlp(const llhip_mlp_in_desc* d, const llhip_resid_desc* r, const void* wd_panel, void* wd_acc,
                  int64_t R, int64_t N_out, void* stream);

/* golden.py:316-342 + 124-137 + 119-120 -- one row of the last down projection finished from its
 * partial sums (r, written to r->x_out), then rmsnorm and quant of it (h_out, hq_out), by one
 * workgroup: the input of llhip_dec_head with pre.prequant set. */
int llhip_dec_finish(const llhip_norm_quant_desc* d, const llhip_resid_desc* r, void* stream);
/* golden.py:286-296 + 316-342 + 376-377 -- llhip_norm_linear for one row.  With keys non-NULL
 * (llhip_dec_head_keys(N) uint64 words), also the first half of the greedy step: keys[t] = the best
 * (value, lowest index) of tile t's 16 columns below vocab, and the row's first vocab values
 * recorded at ring[*step] when *step < ring_cap. */
int llhip_dec_head(const llhip_norm_linear_desc* d, int64_t vocab, void* keys, const int32_t* step, int16_t* ring,
                   int64_t ring_ld, int64_t ring_cap, void* stream);
/* golden.py:376-377 -- the number of greedy keys llhip_dec_head writes for an output of N columns */
int64_t llhip_dec_head_keys(int64_t N);
/* golden.py:376-377 + 411-414 + 369-373 -- the greedy step's second half: *token = the first argmax
 * (the best of nkeys keys), ring_tokens[*step] = token when *step < ring_cap, *pos += 1, *step += 1,
 * and row[0..dim) = embed[token] (the next decode launch's input row). */
int llhip_dec_greedy(const void* keys, int64_t nkeys, int32_t* token, int32_t* pos, int32_t* step,
                     int32_t* ring_tokens, int64_t ring_cap, const int16_t* embed, int64_t dim, int16_t* row,
                     void* stream);
/* golden.py:316-342 + 286-296 + 376-377 + 411-414 + 369-373 -- llhip_dec_finish, llhip_dec_head and
 * llhip_dec_greedy of one row as ONE launch of one workgroup per CU: each workgroup finishes the
 * projection r, normalises and quantises the row (workgroup 0 writes the finished row, h_out and
 * hq_out), computes its share of d's 16-column tiles (logits to d->out when non-NULL, the record
 * row at ring[*step] when *step < ring_cap) and its best (value, lowest index) key; the last
 * workgroup to finish takes the greedy step (token, ring_tokens, pos, step, row = embed[token]).
 * d->pre.prequant = 0, d->M = 1, plain epilogue, K a multiple of 64 up to 1024, vocab <= N; embed
 * holds at least vocab rows of dim i16 values (the token is below vocab).  keys: the
 * launch's llhip_dec_logits_keys() uint64 words, zero-filled before the first launch -- the
 * arrival counter returns to zero at the end of each launch.  Launches sharing keys run in order.
 * panel: NULL, or d->W in tile order, which streams in whole 1 KiB pieces: for 16-column tile t, K
 * step s and lane l = 16 kg + c, bytes [16 l, 16 l + 16) of piece t K/64 + s hold
 * W[16 t + c][64 s + 16 kg, +16) -- ceil(N/16) tiles, columns past N zero. */
int llhip_dec_logits(const llhip_norm_linear_desc* d, const void* panel, const llhip_resid_desc* r, int64_t vocab,
                     void* keys, int32_t* token, int32_t* pos, int32_t* step, int16_t* ring, int64_t ring_ld,
                     int32_t* ring_tokens, int64_t ring_cap, const int16_t* embed, int64_t dim, int16_t* row,
                     void* stream);
/* golden.py:316-342 -- W [N][K] i8 (K a multiple of 64) rewritten in llhip_dec_logits' tile order
 * into panel (ceil(N/16) 16 K bytes) */
int llhip_dec_logits_panel(const void* W, int64_t N, int64_t K, void* panel, void* stream);
/* golden.py:376-377 -- the uint64 words of llhip_dec_logits' keys */
int64_t llhip_dec_logits_keys(void);

/* ---- decode step: every layer of one decode row in one launch ----
 * golden.py:392-397 (decode) running golden.py:275-314 over the layers of a fused graph whose every
 * layer is  rmsnorm, quant, linear q/k/v (+bias), rope q/k, quant q/k, kv_write, attention,
 * linear o (resadd), rmsnorm, quant, linear gate (silu), linear up (mul), quant, linear down
 * (resadd)  -- the layers of the decode chain above, without Q/K norm, head_dim 64.
 * One persistent workgroup per CU computes its fixed share of each stage (q/k/v columns, an
 * attention head slice with its output-projection partial sums, FFN columns with their
 * down-projection partial sums) and hands results to the next stage's workgroups through
 * device-scope flags; each workgroup's weights for a stage are requested before it waits for
 * the stage's input.  Every wait is bounded: a timed-out wait records an error (read with
 * llhip_dec_step_status) and the launch ends.  The KV caches receive the row's keys and values;
 * the last layer's down projection is left as int32 partial sums (llhip_dec_step_outputs) for
 * llhip_dec_finish, with the residual row it adds to.  No other activation is written. */
typedef struct llhip_step_layer {
  const void* g1; int64_t eps1, C1, sh1, Mq1, Sq1; /* attention rmsnorm + quant */
  const void* W[3]; const void* rq[3]; const void* bias[3]; /* q, k, v (bias NULL when absent) */
  int64_t quant_M[2], quant_S[2]; /* quant of rope(q), rope(k) */
  void* kc; void* vc;             /* int8 caches [Hkv][max_seq][D] */
  int64_t Ms, Ss, Mo, So, prob_bits;
  const void* wo_panel;           /* i8 [H][dim][D]: W_o[n][h*D + d] at [h][n][d] */
  const void* rq_o; const void* bias_o;
  const void* g2; int64_t eps2, C2, sh2, Mq2, Sq2; /* mlp rmsnorm + quant */
  const void* Wg; const void* Wu; const void* rqg; const void* rqu; const void* bg; const void* bu;
  int64_t silu_Mi, silu_Si, silu_sh, mul_sh, fq_M, fq_S;
  const void* wd_panel;           /* i8 [F/16][dim][16]: W_d[n][16b + j] at [b][n][j] */
  const void* rq_d; const void* bias_d;
} llhip_step_layer;

typedef struct llhip_dec_step_desc {
  const llhip_step_layer* layers; /* host array of L layers (copied by create) */
  int64_t L, dim, H, Hkv, D, F, max_seq;
  const void* x_in;               /* i16 [dim] the launch's input row */
  const void* cos_tab; const void* sin_tab; /* i16 [max_seq][D/2] */
  const void* pos_dev;            /* int32 device position of the row */
} llhip_dec_step_desc;

typedef struct llhip_dec_step llhip_dec_step;
/* golden.py:246-273 (GoldenModel over the qgraph's layers) -- validate the graph shape and allocate
 * the step's device state (zero-filled).  Returns NULL with llhip_last_error() set when the shape is
 * not supported (head_dim other than 64, dim other than 576/896/1024, more units than CUs, weights,
 * gammas, requant tables, biases or panels not 16-byte aligned). */
llhip_dec_step* llhip_dec_step_create(const llhip_dec_step_desc* d);
/* golden.py:392-397 + 275-314 -- one decode row through every layer (stream-ordered; capturable in a
 * graph).  The row's input is x_in at position *pos_dev. */
int llhip_dec_step_run(llhip_dec_step* s, void* stream);
/* golden.py:316-342 (the last layer's resadd down projection, finished by llhip_dec_finish) -- device
 * pointers valid for the step's lifetime: *acc = int32 [8][dim], its partial sums after a run;
 * *resid = i16 [dim], the residual row it adds to. */
int llhip_dec_step_outputs(llhip_dec_step* s, void** acc, void** resid);
/* golden.py:392-397 -- synchronous: *launches = completed launches, *err = nonzero when a launch hit
 * a bounded-wait timeout (sticky: later launches end at once). */
int llhip_dec_step_status(llhip_dec_step* s, int64_t* launches, int64_t* err);
/* golden.py:246-273 -- release what llhip_dec_step_create allocated. */
void llhip_dec_step_destroy(llhip_dec_step* s);

/* ---- the reference accelerator's instruction set on the GPU ----
 * A device holding the ISA's DRAM and 1 MiB SRAM in GPU memory that runs .llbin programs (docs/ISA.md,
 * binary version 2) with the functional simulator's semantics and performance counters.  Errors
 * (the simulator's runtime_error conditions, with its messages) return a negative errno with the
 * message in llhip_last_error().  Calls on one device must not overlap (one host thread at a time). */
typedef struct llhip_device llhip_device;
#define LLHIP_DEV_NUM_PERF 27

/* runtime/include/llaccel/device.h:41 makeFuncSim (funcsim.cpp:24-27): a device with max(dram_bytes,
 * 1 MiB) of zeroed DRAM; epilogue_fusion selects the v2 target (GEMM epilogues allowed).  NULL on
 * failure. */
llhip_device* llhip_dev_create(uint64_t dram_bytes, int epilogue_fusion);
/* device.h:17 ~Device */
void llhip_dev_destroy(llhip_device* dev);
/* device.h:22 dramWrite (funcsim.cpp:29-33): host bytes into DRAM, which grows to addr + n */
int llhip_dev_dram_write(llhip_device* dev, uint64_t addr, const void* src, uint64_t n);
/* device.h:23 dramRead (funcsim.cpp:34-37) */
int llhip_dev_dram_read(llhip_device* dev, uint64_t addr, void* dst, uint64_t n);
/* device.h:24 dramSize */
uint64_t llhip_dev_dram_size(const llhip_device* dev);
/* device.h:26 run (funcsim.cpp:41-107, sequential policy): executes from pc until HALT with the POS
 * register at pos; perf (27 counters, include/llaccel/isa.h:133-141) may be NULL. */
int llhip_dev_run(llhip_device* dev, uint32_t pc, uint32_t pos, uint64_t* perf);
/* device.h:28 sramSnapshot: the 1 MiB SRAM into dst */
int llhip_dev_sram_snapshot(llhip_device* dev, void* dst);
/* device.h:36 DeviceOptions::interleaveSeed (funcsim.cpp:47-90): 0 runs the sequential policy;
 * another seed executes the engine queues in the simulator's random legal order for that seed
 * (std::mt19937 + uniform_int_distribution), which exposes missing semaphore dependencies. */
int llhip_dev_set_interleave(llhip_device* dev, uint32_t seed);
/* device.h:19 maxAttentionHeadDim (funcsim.cpp:24) */
uint32_t llhip_dev_max_attention_head_dim(void);
/* device.h:22 (device side): the DRAM's device address, valid until the DRAM next grows */
void* llhip_dev_dram_ptr(llhip_device* dev);

/* ---- float side: activation calibration and SmoothQuant over fp32 tensors on the GPU ---- */
/* calibrate.py:56-66 (AbsMaxRecorder.run_node), smoothquant.py:95-99 (recorder): running maxima of
 * |x| over the rows of x [rows][ld] -- per column into col_max [cols] and over the tensor into
 * amax [1] (either may be NULL; both start at the caller's values, 0 for a fresh record).  Exact in
 * any order.  Non-finite values are not folded in but counted into nonfinite [1]. */
int llhip_f32_absmax(const float* x, int64_t rows, int64_t cols, int64_t ld, float* col_max, float* amax,
                     int32_t* nonfinite, void* stream);
/* calibrate.py:67-72: out_min [1] = min(out_min, min over the rows of x [rows][width] of
 * sqrt(mean(x^2))), in double */
int llhip_f32_rms_min(const float* x, int64_t rows, int64_t width, double* out_min, void* stream);
/* smoothquant.py:250-261: x [rows][ld] in place: x * col_mul[c], then / col_div[c], then / row_div[r],
 * each an fp32 operation (NULL skips one) */
int llhip_f32_rescale(float* x, int64_t rows, int64_t cols, int64_t ld, const float* col_mul, const float* col_div,
                      const float* row_div, void* stream);
/* smoothquant.py:152-163 (quantization_objective, weight terms): out [2] += the sums over W [rows][cols]
 * (rows of cols floats) of w^2 * act_err[c] and (q - w)^2 * act_energy[c], w = W * scales[c], q = w
 * rounded to the row's int8 grid max|w| / 127 (half to even, clamped to [-128, 127]) */
int llhip_f32_smooth_objective(const float* W, int64_t rows, int64_t cols, const float* scales, const float* act_err,
                               const float* act_energy, double* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
