/*
 * q4kv_oracle.h -- CPU restatement of SuzuQu-Engine's QSA KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or as the timed CPU baseline). The product library (libq4kv.so) never
 * links, loads or calls it.
 *
 * Every function cites the reference file:line it restates. Reference paths
 * are relative to the upstream tree (src/...).
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   orc_f16_from_f32   exhaustive against x86 F16C (_cvtss_sh, RNE) over all
 *                      2^32 float bit patterns minus NaNs, sampled; and the
 *                      round-trip f16->f32->f16 identity on all 65536 codes.
 *   orc_f16_to_f32     all 65536 codes against the reference's own
 *                      q4_f16_to_f32 (oracle/_ref build of src/q4_quant.c).
 *   orc_quant_q8_0     closed forms (zero block, ramp block, single +-1 value),
 *                      invariants (|q|<=127, |q*d-x|<=d/2 (+1ulp), argmax->+-127),
 *                      dequant round trip through the reference's
 *                      q4_dequant_row(Q8_0) from oracle/_ref.
 *   orc_dequant_q8_0   against q4_dequant_row(Q4_T_Q8_0) from oracle/_ref.
 *   orc_attn           the reference's own known-answer test inputs
 *                      (src/q4_test.c:134-238) and closed forms: width-1 list
 *                      returns V exactly, equal scores give the mean of V, an
 *                      all -1 list gives 0, permutation invariance of the list,
 *                      causal dense == indexed list 0..t, gate=0 halves output.
 *   orc_qsa_topk       an independent sort-based brute force (numpy, stable
 *                      argsort on (key desc, index asc)) over random, tied,
 *                      +-0, NaN and dense-prefix rows; orc_qsa_key against
 *                      numpy float ordering.
 *   orc_qsa_pool       closed forms: constant raw keys pool to wn * sign
 *   orc_qsa_prep         (RMSNorm of a constant), RoPE preserves each pair's
 *                      norm and is the identity at position 0 and for dims
 *                      >= n_rot; a single-pair input rotates by the angle
 *                      formed from orc_rope_freq, which is checked against
 *                      numpy float32 arithmetic.
 *   orc_qsa_score      numpy float64 einsum + relu + -1e30 mask.
 *   orc_gemv_q8_0      the reference's own q4_dequant_row (oracle/_ref) times x
 *                      in float64 (an independent dequantisation), and closed
 *                      forms: identity-like weights pick one column of x.
 */
#ifndef Q4KV_ORACLE_H
#define Q4KV_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KV widths, as src/q4_fwd.c:637-642 (kv_kind_of): 0 f32, 1 f16, 2 q8_0. */
enum { ORC_KV_F32 = 0, ORC_KV_F16 = 1, ORC_KV_Q8 = 2 };

uint16_t orc_f16_from_f32(float x);
float orc_f16_to_f32(uint16_t h);

/* fp32 [n] -> q8_0 blocks (n % 32 == 0), 34 B per block. */
int orc_quant_q8_0(const float *x, uint64_t n, uint8_t *out);
/* fp32 [n] -> fp16 [n] (RNE). */
void orc_quant_f16(const float *x, uint64_t n, uint16_t *out);
/* q8_0 blocks -> fp32 [n]. */
void orc_dequant_q8_0(const uint8_t *src, uint64_t n, float *dst);

/* Bytes per token of one K (or V) cache, src/q4_fwd.c:644-650. */
uint32_t orc_kv_token_bytes(int kind, uint32_t n_kvh, uint32_t hd);
/* Width tag of a session image, src/q4_fwd.c:663-665. */
uint32_t orc_kv_tag(int kind);

/* Append one token's K and V rows (n = n_kvh*hd floats each) at token
 * position pos of caches with bpt bytes per token (src/q4_rocm.cu:7962-8000). */
int orc_kv_append(uint8_t *kc, uint8_t *vc, const float *k, const float *v,
                  uint32_t n, uint32_t bpt, int kind, uint32_t pos);

/*
 * Gated GQA attention over a K/V cache of any width.
 *   q    [n_tok][n_head][hd]       gate [n_tok][n_head][hd] or NULL (identity)
 *   out  [n_tok][n_head][hd]
 * Position list for (token t, kv head kh):
 *   idx == NULL : dense causal prefix 0 .. min(kv_base+t+1, max_kv)-1
 *   idx != NULL : idx[t*tok_stride + kh*kvh_stride + j], j < width, -1 = pad
 * Precision: dbl != 0 accumulates in double (the golden reference);
 * dbl == 0 is fp32 throughout, the shape of src/q4_fwd.c:330-407 (timed
 * CPU baseline). nthreads > 1 splits (token, head) pairs over OpenMP.
 */
int orc_attn(const float *q, const void *kcache, const void *vcache, int kind,
             const float *gate, float *out, uint32_t n_head, uint32_t n_kvh,
             uint32_t hd, uint32_t n_tok, const int32_t *idx, uint32_t width,
             uint64_t tok_stride, uint64_t kvh_stride, uint32_t kv_base,
             uint32_t max_kv, float scale, int dbl, int nthreads);

/* q8_0 GEMV y = scale * W x, W [nrows][ncols/32 blocks] (src/q4_rocm.cu:1262-1285). */
int orc_gemv_q8_0(const uint8_t *w, uint64_t nrows, uint64_t ncols, const float *x, float *y,
                  float scale);

/* ---- QSA indexer and Q/K preparation (oracle/qsa_index_oracle.c) ---- */
/* Order-preserving key of an fp32 score, src/q4_rocm.cu:7471-7474. */
uint32_t orc_qsa_key(float f);
/* fp32 RoPE frequency base^-(p/np), correctly rounded. */
float orc_rope_freq(float base, uint32_t p, uint32_t np);
/* One head: RMSNorm * wn then RoPE of dims < n_rot at pos
 * (src/q4_rocm.cu:6229-6289). */
int orc_qsa_prep(const float *src, float *dst, const float *wn, uint32_t hd,
                 uint32_t n_rot, int32_t pos, float base, float eps);
/* Pool blocks [b0, b1) of fp16 raw keys (src/q4_rocm.cu:7366-7401). */
int orc_qsa_pool(const uint16_t *raw, float *pool, const float *wn, uint32_t hd,
                 uint32_t ratio, uint32_t b0, uint32_t b1, uint32_t n_rot,
                 float base, float eps);
/* Block scores per token (src/q4_rocm.cu:7412-7445). */
int orc_qsa_score(const float *q, const float *pool, float *score, uint32_t n_tok,
                  uint32_t n_blocks, uint32_t stride, uint32_t n_head, uint32_t hd,
                  uint32_t pos0, uint32_t ratio);
/* Exact top-k block selection and expansion (src/q4_rocm.cu:7722-7846). */
int orc_qsa_topk(const float *score, int32_t *sel, uint32_t n_tok, uint32_t stride,
                 uint32_t k_blk, uint32_t ratio, uint32_t pos0, uint32_t width);

#ifdef __cplusplus
}
#endif
#endif
