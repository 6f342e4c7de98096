/*
 * qr_oracle.h -- CPU oracle for the paged-KV attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped.  The product path (libqr_attn.so)
 * neither links nor calls anything here.
 *
 * Two families of functions:
 *   qro_*      op-order-faithful restatements of the reference's C#
 *              arithmetic (Vector256 multiply-then-add with no FMA, lane sums
 *              in lane order 0..7, platform expf, sequential fp32 softmax
 *              sum).  Built with -ffp-contract=off so gcc never fuses a
 *              multiply into an add.
 *   qro_*_f64  textbook fp64 formulas used to attribute errors.
 *
 * Reference paths are relative to the QuantRunner source tree
 * (Core = src/QuantRunner.Core).
 */
#ifndef QR_ORACLE_H
#define QR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- 16-bit codecs: Core/Dtypes.cs:76-139 ---- */
float    qro_f16_to_f32(uint16_t h);          /* Dtypes.cs:76-97  (exact)              */
uint16_t qro_f32_to_f16(float f);             /* Dtypes.cs:100-126 (half-away in normal range) */
float    qro_bf16_to_f32(uint16_t b);         /* Dtypes.cs:129    (exact)              */
uint16_t qro_f32_to_bf16(float f);            /* Dtypes.cs:132-139 (round-nearest-even) */
void qro_f16_to_f32_n(const uint16_t* src, float* dst, long n);
void qro_f32_to_f16_n(const float* src, uint16_t* dst, long n);
void qro_bf16_to_f32_n(const uint16_t* src, float* dst, long n);
void qro_f32_to_bf16_n(const float* src, uint16_t* dst, long n);

/* ---- primitives: Core/Kernels/SimdMath.cs, Core/Kernels/TransformerOps.cs ---- */
float qro_dot_f32(const float* a, const float* b, int n);              /* SimdMath.cs:34-53 */
void  qro_axpy_f32(const float* x, float* y, float alpha, int n);      /* SimdMath.cs:55-71 */
void  qro_softmax(float* x, int n);                                    /* TransformerOps.cs:92-107 */
void  qro_build_cos_sin(long pos, int head_dim, float theta, float* row); /* TransformerOps.cs:56-66 */
void  qro_rope(float* q, float* k, const float* cos_sin, int nq, int nk, int head_dim); /* :69-88 */
/* Applies RoPE to `rows` rows of `width` floats; row r is at position pos0 + r. */
void  qro_rope_rows(float* x, long rows, int width, int head_dim, long pos0, float theta);

/* ---- GQA decode attention: Core/Runtime/PagedKvCache.cs:83-136 ----
 * K and V are token-major fp32 rows [seq][kv_heads*head_dim] (the reference
 * walks pages in token order, so paging does not change the op order).
 * scores: caller scratch of heads*seq floats.                              */
void qro_kv_attention(const float* K, const float* V, int seq, int heads, int kv_heads,
                      int head_dim, const float* q, float* attn, float scale, float* scores);
/* textbook softmax(q K^T * scale) V in fp64, same GQA map kvh = h*kv_heads/heads */
void qro_kv_attention_f64(const float* K, const float* V, int seq, int heads, int kv_heads,
                          int head_dim, const float* q, double* attn, double scale);

/* ---- MLA absorbed attention: Core/Runtime/StreamingEngine.cs:508-577 ----
 * lat: [seq][kv_lora+rope] latent rows; q_tilde [heads][kv_lora]; q_rope [heads][rope];
 * u [heads][kv_lora].  scores: caller scratch of seq floats.             */
void qro_mla_attention(const float* lat, int seq, int kv_lora, int rope, int heads,
                       const float* q_tilde, const float* q_rope, float scale, float* u,
                       float* scores);
void qro_mla_attention_f64(const float* lat, int seq, int kv_lora, int rope, int heads,
                           const float* q_tilde, const float* q_rope, double scale, double* u);
/* q-absorb, StreamingEngine.cs:517-529: q [heads][nope+rope], kvb [heads*(nope+vdim)][kv_lora] */
void qro_mla_q_absorb(const float* q, const float* kvb, int heads, int nope, int rope, int vdim,
                      int kv_lora, float* q_tilde);
/* W_UV up-projection, StreamingEngine.cs:569-576: out [heads][vdim] */
void qro_mla_wuv(const float* u, const float* kvb, int heads, int nope, int vdim, int kv_lora,
                 float* out);
/* expanded-K/V fp64 attention, the comparison of Cli/Commands.cs:2065-2152 extended with rope */
void qro_mla_expanded_f64(const float* q, const float* kvb, const float* lat, int seq, int heads,
                          int nope, int rope, int vdim, int kv_lora, double scale, double* out);

/* ---- weight rows: Core/Quantization/BlockDequantizer.cs ----
 * fmt is a QuantFormat value (Dtypes.cs:6-26).  Supported here: F32 0, F16 1,
 * BF16 2, Q4_0 3, Q8_0 4, Q4_K 6, Q6_K 7.
 * qro_row_bytes: bytes of n weights (Dtypes.cs:38-50 block specs), -1 when the
 * format is unsupported or n is not a whole number of blocks.
 * qro_dequant_row: decodes n weights; returns 0, or -1 as above.           */
long qro_row_bytes(int fmt, long n);
int  qro_dequant_row(int fmt, const uint8_t* src, long n, float* dst);

/* ---- fused dequant + dot: Core/Kernels/DotKernels.cs ----
 * qro_dot_row: DotRow (:24-46) for the formats above, in each format's own operation
 * order (:52-447).  qro_matvec: MatVec (:599-608), y[r] = DotRow(row r, x); -1 when the
 * format cannot hold rows of `cols` weights.                                      */
float qro_dot_row(int fmt, const uint8_t* w, const float* x, int cols);
int   qro_matvec(int fmt, const uint8_t* w, long rows, int cols, const float* x, float* y);

#ifdef __cplusplus
}
#endif
#endif
