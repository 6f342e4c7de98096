/*
 * qr_oracle.c -- CPU oracle for the paged-KV attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker; see qr_oracle.h).  Each function
 * restates the reference's arithmetic from its semantics and cites the
 * reference lines it follows.  Compile with -ffp-contract=off: the reference
 * runs on RyuJIT, which never contracts a multiply and an add into an FMA, and
 * Vector256.Multiply / Vector256.Add are separately rounded IEEE operations.
 */
#include "qr_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef __AVX2__
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------- */
/* 16-bit codecs                                                             */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Dtypes.cs:76-97: exact widening; subnormal halves are renormalised. */
float qro_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* shift the mantissa up until its leading one reaches bit 10 */
        int shifts = 0;
        while ((m & 0x400u) == 0) { m <<= 1; shifts++; }
        /* value = 1.m' * 2^(-14 - shifts) */
        return u2f(sign | ((uint32_t)(127 - 14 - shifts) << 23) | ((m & 0x3FFu) << 13));
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* Dtypes.cs:100-126.  Normal range: add half an ulp (0x1000) to the 23-bit
 * mantissa and truncate (ties round away from zero, :111-113).  Subnormal
 * range: round-nearest-even on the shifted-out bits (:118-125). */
uint16_t qro_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t biased = (x >> 23) & 0xFFu;
    int e = (int)biased - 127;
    uint32_t man = x & 0x7FFFFFu;
    if (biased == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    if (e >= -14) {
        uint32_t r = man + 0x1000u;
        if (r & 0x800000u) { r = 0; e++; }
        return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | (r >> 13));
    }
    if (e < -25) return (uint16_t)sign;
    {
        uint32_t full = 0x800000u | man;
        int shift = (-e - 14) + 13;                 /* 14..24 */
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
}

/* Dtypes.cs:129 */
float qro_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* Dtypes.cs:132-139: add 0x7FFF plus the kept lsb, keep the high half. */
uint16_t qro_f32_to_bf16(float f)
{
    uint32_t x = f2u(f);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

void qro_f16_to_f32_n(const uint16_t* s, float* d, long n) { for (long i = 0; i < n; i++) d[i] = qro_f16_to_f32(s[i]); }
void qro_f32_to_f16_n(const float* s, uint16_t* d, long n) { for (long i = 0; i < n; i++) d[i] = qro_f32_to_f16(s[i]); }
void qro_bf16_to_f32_n(const uint16_t* s, float* d, long n) { for (long i = 0; i < n; i++) d[i] = qro_bf16_to_f32(s[i]); }
void qro_f32_to_bf16_n(const float* s, uint16_t* d, long n) { for (long i = 0; i < n; i++) d[i] = qro_f32_to_bf16(s[i]); }

/* ------------------------------------------------------------------------- */
/* primitives                                                                */
/* ------------------------------------------------------------------------- */

/* SimdMath.cs:34-53 with HSum :17-22.  For n >= 8: eight lane accumulators,
 * acc = acc + (a*b) per 8-wide block, then lanes summed 0..7 into a scalar
 * starting at 0, then the scalar tail.  For n < 8: a plain scalar loop. */
float qro_dot_f32(const float* a, const float* b, int n)
{
    if (n >= 8) {
        int i = 0;
        float lanes[8];
#ifdef __AVX2__
        __m256 acc = _mm256_setzero_ps();
        for (; i + 8 <= n; i += 8)
            acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i)));
        _mm256_storeu_ps(lanes, acc);
#else
        for (int j = 0; j < 8; j++) lanes[j] = 0.0f;
        for (; i + 8 <= n; i += 8)
            for (int j = 0; j < 8; j++) {
                float p = a[i + j] * b[i + j];
                lanes[j] = lanes[j] + p;
            }
#endif
        float s = 0.0f;
        for (int j = 0; j < 8; j++) s += lanes[j];
        for (; i < n; i++) s += a[i] * b[i];
        return s;
    }
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* SimdMath.cs:55-71: y = y + alpha*x, product rounded before the add. */
void qro_axpy_f32(const float* x, float* y, float alpha, int n)
{
    int i = 0;
    if (n >= 8) {
#ifdef __AVX2__
        __m256 va = _mm256_set1_ps(alpha);
        for (; i + 8 <= n; i += 8)
            _mm256_storeu_ps(y + i, _mm256_add_ps(_mm256_loadu_ps(y + i),
                                                  _mm256_mul_ps(va, _mm256_loadu_ps(x + i))));
#else
        for (; i + 8 <= n; i += 8)
            for (int j = 0; j < 8; j++) {
                float p = alpha * x[i + j];
                y[i + j] = y[i + j] + p;
            }
#endif
    }
    for (; i < n; i++) y[i] += alpha * x[i];
}

/* TransformerOps.cs:92-107: max from float.MinValue, exp(x - max) with a
 * sequential fp32 sum, one reciprocal, then scale every entry by it. */
void qro_softmax(float* x, int n)
{
    float mx = -FLT_MAX;
    for (int i = 0; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* TransformerOps.cs:56-66: freq_i = theta^(-2i/D) evaluated in fp32,
 * angle = (float)pos * freq_i; row = [cos..., sin...]. */
void qro_build_cos_sin(long pos, int head_dim, float theta, float* row)
{
    int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        float ex = (-2.0f * (float)i) / (float)head_dim;
        float freq = powf(theta, ex);
        float ang = (float)pos * freq;
        row[i] = cosf(ang);
        row[half + i] = sinf(ang);
    }
}

/* TransformerOps.cs:69-88: rotate-half on every head of q and k. */
static void rope_head(float* v, const float* cs, int half)
{
    for (int i = 0; i < half; i++) {
        float c = cs[i], s = cs[half + i];
        float x0 = v[i], x1 = v[i + half];
        v[i] = x0 * c - x1 * s;
        v[i + half] = x0 * s + x1 * c;
    }
}

void qro_rope(float* q, float* k, const float* cs, int nq, int nk, int head_dim)
{
    int half = head_dim / 2;
    for (int off = 0; off < nq; off += head_dim) rope_head(q + off, cs, half);
    for (int off = 0; off < nk; off += head_dim) rope_head(k + off, cs, half);
}

void qro_rope_rows(float* x, long rows, int width, int head_dim, long pos0, float theta)
{
    float* cs = (float*)malloc(sizeof(float) * (size_t)head_dim);
    for (long r = 0; r < rows; r++) {
        qro_build_cos_sin(pos0 + r, head_dim, theta, cs);
        qro_rope(x + r * (long)width, NULL, cs, width, 0, head_dim);
    }
    free(cs);
}

/* ------------------------------------------------------------------------- */
/* GQA decode attention                                                      */
/* ------------------------------------------------------------------------- */

/* PagedKvCache.cs:83-136.
 * pass 1 (:91-109): positions in order, heads in order:
 *     sc[h][p] = DotF32(q_h, K[p] + kvh*D) * scale,  kvh = h*kv_heads/heads (:103)
 * pass 2 (:112-134): per head: Softmax(sc_h, seq); dst = 0;
 *     for p in order: AxpyF32(V[p] + kvh*D, dst, sc_h[p]). */
void qro_kv_attention(const float* K, const float* V, int seq, int heads, int kv_heads,
                      int head_dim, const float* q, float* attn, float scale, float* scores)
{
    const long kv_dim = (long)kv_heads * head_dim;
    for (int p = 0; p < seq; p++) {
        const float* krow = K + (long)p * kv_dim;
        for (int h = 0; h < heads; h++) {
            int kvh = (int)((long)h * kv_heads / heads);
            scores[(long)h * seq + p] =
                qro_dot_f32(q + (long)h * head_dim, krow + (long)kvh * head_dim, head_dim) * scale;
        }
    }
    for (int h = 0; h < heads; h++) {
        float* sc = scores + (long)h * seq;
        qro_softmax(sc, seq);
        float* dst = attn + (long)h * head_dim;
        for (int i = 0; i < head_dim; i++) dst[i] = 0.0f;
        int kvh = (int)((long)h * kv_heads / heads);
        for (int p = 0; p < seq; p++)
            qro_axpy_f32(V + (long)p * kv_dim + (long)kvh * head_dim, dst, sc[p], head_dim);
    }
}

void qro_kv_attention_f64(const float* K, const float* V, int seq, int heads, int kv_heads,
                          int head_dim, const float* q, double* attn, double scale)
{
    const long kv_dim = (long)kv_heads * head_dim;
    double* s = (double*)malloc(sizeof(double) * (size_t)(seq > 0 ? seq : 1));
    for (int h = 0; h < heads; h++) {
        int kvh = (int)((long)h * kv_heads / heads);
        const float* qh = q + (long)h * head_dim;
        double mx = -INFINITY;
        for (int p = 0; p < seq; p++) {
            const float* kr = K + (long)p * kv_dim + (long)kvh * head_dim;
            double d = 0.0;
            for (int i = 0; i < head_dim; i++) d += (double)qh[i] * (double)kr[i];
            s[p] = d * scale;
            if (s[p] > mx) mx = s[p];
        }
        double sum = 0.0;
        for (int p = 0; p < seq; p++) { s[p] = exp(s[p] - mx); sum += s[p]; }
        double* o = attn + (long)h * head_dim;
        for (int i = 0; i < head_dim; i++) o[i] = 0.0;
        for (int p = 0; p < seq; p++) {
            const float* vr = V + (long)p * kv_dim + (long)kvh * head_dim;
            double w = s[p] / sum;
            for (int i = 0; i < head_dim; i++) o[i] += w * (double)vr[i];
        }
    }
    free(s);
}

/* ------------------------------------------------------------------------- */
/* MLA absorbed attention                                                    */
/* ------------------------------------------------------------------------- */

/* StreamingEngine.cs:531-568 for each head h:
 *   s_t = DotF32(q~_h, c_t[0:kv_lora]) (+ DotF32(q_rope_h, c_t[kv_lora:]) if rope > 0)
 *   sc[t] = s_t * scale;  Softmax(sc, seq)
 *   u_h = 0;  for t in order: AxpyF32(c_t[0:kv_lora], u_h, sc[t]). */
void qro_mla_attention(const float* lat, int seq, int kv_lora, int rope, int heads,
                       const float* q_tilde, const float* q_rope, float scale, float* u,
                       float* scores)
{
    const long ld = (long)kv_lora + rope;
    for (int h = 0; h < heads; h++) {
        const float* qt = q_tilde + (long)h * kv_lora;
        const float* qr = q_rope + (long)h * rope;
        for (int t = 0; t < seq; t++) {
            const float* ct = lat + (long)t * ld;
            float s = qro_dot_f32(qt, ct, kv_lora);
            if (rope > 0) s += qro_dot_f32(qr, ct + kv_lora, rope);
            scores[t] = s * scale;
        }
        qro_softmax(scores, seq);
        float* uh = u + (long)h * kv_lora;
        for (int k = 0; k < kv_lora; k++) uh[k] = 0.0f;
        for (int t = 0; t < seq; t++) qro_axpy_f32(lat + (long)t * ld, uh, scores[t], kv_lora);
    }
}

void qro_mla_attention_f64(const float* lat, int seq, int kv_lora, int rope, int heads,
                           const float* q_tilde, const float* q_rope, double scale, double* u)
{
    const long ld = (long)kv_lora + rope;
    double* s = (double*)malloc(sizeof(double) * (size_t)(seq > 0 ? seq : 1));
    for (int h = 0; h < heads; h++) {
        const float* qt = q_tilde + (long)h * kv_lora;
        const float* qr = q_rope + (long)h * rope;
        double mx = -INFINITY;
        for (int t = 0; t < seq; t++) {
            const float* ct = lat + (long)t * ld;
            double d = 0.0;
            for (int k = 0; k < kv_lora; k++) d += (double)qt[k] * (double)ct[k];
            for (int r = 0; r < rope; r++) d += (double)qr[r] * (double)ct[kv_lora + r];
            s[t] = d * scale;
            if (s[t] > mx) mx = s[t];
        }
        double sum = 0.0;
        for (int t = 0; t < seq; t++) { s[t] = exp(s[t] - mx); sum += s[t]; }
        double* uh = u + (long)h * kv_lora;
        for (int k = 0; k < kv_lora; k++) uh[k] = 0.0;
        for (int t = 0; t < seq; t++) {
            double w = s[t] / sum;
            const float* ct = lat + (long)t * ld;
            for (int k = 0; k < kv_lora; k++) uh[k] += w * (double)ct[k];
        }
    }
    free(s);
}

/* StreamingEngine.cs:517-529: q~_h[k] = sum_j q_h[j] * W_kvb[h*(nope+vdim)+j][k],
 * accumulated j = 0..nope-1 with a separately rounded product per step. */
void qro_mla_q_absorb(const float* q, const float* kvb, int heads, int nope, int rope, int vdim,
                      int kv_lora, float* q_tilde)
{
    const int per_head = nope + vdim, qk = nope + rope;
    for (int h = 0; h < heads; h++) {
        float* qt = q_tilde + (long)h * kv_lora;
        for (int k = 0; k < kv_lora; k++) qt[k] = 0.0f;
        for (int j = 0; j < nope; j++) {
            const float* row = kvb + ((long)h * per_head + j) * kv_lora;
            float qv = q[(long)h * qk + j];
            for (int k = 0; k < kv_lora; k++) { float p = qv * row[k]; qt[k] = qt[k] + p; }
        }
    }
}

/* StreamingEngine.cs:569-576: out_h[j] = DotF32(W_kvb[h*(nope+vdim)+nope+j], u_h). */
void qro_mla_wuv(const float* u, const float* kvb, int heads, int nope, int vdim, int kv_lora,
                 float* out)
{
    const int per_head = nope + vdim;
    for (int h = 0; h < heads; h++)
        for (int j = 0; j < vdim; j++)
            out[(long)h * vdim + j] =
                qro_dot_f32(kvb + ((long)h * per_head + nope + j) * kv_lora, u + (long)h * kv_lora, kv_lora);
}

/* Cli/Commands.cs:2065-2152 (naive side), extended with the decoupled rope key:
 *   K_t,h[j] = W_UK,h[j] . c_t,  V_t,h[j] = W_UV,h[j] . c_t
 *   score = (q_nope . K_t,h + q_rope . k_pe_t) * scale;  out = softmax . V */
void qro_mla_expanded_f64(const float* q, const float* kvb, const float* lat, int seq, int heads,
                          int nope, int rope, int vdim, int kv_lora, double scale, double* out)
{
    const int per_head = nope + vdim, qk = nope + rope;
    const long ld = (long)kv_lora + rope;
    double* s = (double*)malloc(sizeof(double) * (size_t)(seq > 0 ? seq : 1));
    for (int h = 0; h < heads; h++) {
        const float* qh = q + (long)h * qk;
        double mx = -INFINITY;
        for (int t = 0; t < seq; t++) {
            const float* ct = lat + (long)t * ld;
            double d = 0.0;
            for (int j = 0; j < nope; j++) {
                const float* row = kvb + ((long)h * per_head + j) * kv_lora;
                double kj = 0.0;
                for (int k = 0; k < kv_lora; k++) kj += (double)row[k] * (double)ct[k];
                d += (double)qh[j] * kj;
            }
            for (int r = 0; r < rope; r++) d += (double)qh[nope + r] * (double)ct[kv_lora + r];
            s[t] = d * scale;
            if (s[t] > mx) mx = s[t];
        }
        double sum = 0.0;
        for (int t = 0; t < seq; t++) { s[t] = exp(s[t] - mx); sum += s[t]; }
        for (int j = 0; j < vdim; j++) {
            const float* row = kvb + ((long)h * per_head + nope + j) * kv_lora;
            double acc = 0.0;
            for (int t = 0; t < seq; t++) {
                const float* ct = lat + (long)t * ld;
                double vj = 0.0;
                for (int k = 0; k < kv_lora; k++) vj += (double)row[k] * (double)ct[k];
                acc += s[t] / sum * vj;
            }
            out[(long)h * vdim + j] = acc;
        }
    }
    free(s);
}

/* ------------------------------------------------------------------------- */
/* Weight-row decoders: Core/Quantization/BlockDequantizer.cs                */
/* ------------------------------------------------------------------------- */

/* Dtypes.cs:38-50: (weights per block, bytes per block). */
static int fmt_spec(int fmt, int* bs, int* bb)
{
    switch (fmt) {
    case 0: *bs = 1; *bb = 4; return 0;     /* F32  */
    case 1: *bs = 1; *bb = 2; return 0;     /* F16  */
    case 2: *bs = 1; *bb = 2; return 0;     /* BF16 */
    case 3: *bs = 32; *bb = 20; return 0;   /* Q4_0: f16 d, 16 nibble bytes, 2 pad bytes */
    case 4: *bs = 32; *bb = 34; return 0;   /* Q8_0: f16 d, 32 int8 */
    case 6: *bs = 256; *bb = 144; return 0; /* Q4_K */
    case 7: *bs = 256; *bb = 210; return 0; /* Q6_K */
    default: return -1;
    }
}

long qro_row_bytes(int fmt, long n)
{
    int bs, bb;
    if (fmt_spec(fmt, &bs, &bb) || n < 0 || n % bs) return -1;
    return n / bs * bb;
}

static inline uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* BlockDequantizer.cs:155-166 (ggml get_scale_min_k4): 6-bit scale and min of sub-block j. */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

int qro_dequant_row(int fmt, const uint8_t* s, long n, float* y)
{
    if (qro_row_bytes(fmt, n) < 0) return -1;
    switch (fmt) {
    case 0: /* BlockDequantizer.cs:14 */
        memcpy(y, s, (size_t)n * 4);
        return 0;
    case 1: /* :34-41 */
        for (long i = 0; i < n; i++) y[i] = qro_f16_to_f32(le16(s + 2 * i));
        return 0;
    case 2: /* :43-50 */
        for (long i = 0; i < n; i++) y[i] = qro_bf16_to_f32(le16(s + 2 * i));
        return 0;
    case 3: /* :52-69: low nibble -> weight i, high nibble -> weight i+16 */
        for (long b = 0; b < n / 32; b++, s += 20, y += 32) {
            float d = qro_f16_to_f32(le16(s));
            for (int i = 0; i < 16; i++) {
                y[i] = d * (float)((s[2 + i] & 0xF) - 8);
                y[i + 16] = d * (float)((s[2 + i] >> 4) - 8);
            }
        }
        return 0;
    case 4: /* :71-84 */
        for (long b = 0; b < n / 32; b++, s += 34, y += 32) {
            float d = qro_f16_to_f32(le16(s));
            for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)s[2 + i];
        }
        return 0;
    case 6: /* :168-196: d @0, dmin @2, packed scales @4, nibbles @16 (sub-block pairs share 32 bytes) */
        for (long b = 0; b < n / 256; b++, s += 144, y += 256) {
            float d = qro_f16_to_f32(le16(s)), dmin = qro_f16_to_f32(le16(s + 2));
            for (int sub = 0; sub < 8; sub++) {
                int sc, mi;
                scale_min_k4(sub, s + 4, &sc, &mi);
                float a = d * (float)sc, m = dmin * (float)mi;
                const uint8_t* qb = s + 16 + (sub / 2) * 32;
                for (int i = 0; i < 32; i++) {
                    int qv = (sub & 1) ? (qb[i] >> 4) : (qb[i] & 0xF);
                    float t = a * (float)qv;
                    y[sub * 32 + i] = t - m;
                }
            }
        }
        return 0;
    case 7: /* :228-256: ql @0, qh @128, int8 scales @192, d @208 */
        for (long b = 0; b < n / 256; b++, s += 210, y += 256) {
            float d = qro_f16_to_f32(le16(s + 208));
            const uint8_t *ql = s, *qh = s + 128, *sc = s + 192;
            for (int h = 0; h < 256; h += 128) {
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = (ql[h / 2 + l] & 0xF) | (((qh[h / 4 + l] >> 0) & 3) << 4);
                    int q2 = (ql[h / 2 + l + 32] & 0xF) | (((qh[h / 4 + l] >> 2) & 3) << 4);
                    int q3 = (ql[h / 2 + l] >> 4) | (((qh[h / 4 + l] >> 4) & 3) << 4);
                    int q4 = (ql[h / 2 + l + 32] >> 4) | (((qh[h / 4 + l] >> 6) & 3) << 4);
                    const int8_t* scs = (const int8_t*)sc + 8 * (h / 128) + is;
                    y[h + l] = (d * (float)scs[0]) * (float)(q1 - 32);
                    y[h + l + 32] = (d * (float)scs[2]) * (float)(q2 - 32);
                    y[h + l + 64] = (d * (float)scs[4]) * (float)(q3 - 32);
                    y[h + l + 96] = (d * (float)scs[6]) * (float)(q4 - 32);
                }
            }
        }
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------------- */
/* Fused dequant + dot rows: Core/Kernels/DotKernels.cs                       */
/* ------------------------------------------------------------------------- */

/* SimdMath.cs:17-22: lane sum in lane order. */
static float hsum8(const float* v)
{
    float s = 0.0f;
    for (int i = 0; i < 8; i++) s += v[i];
    return s;
}

/* DotKernels.cs:86-100 (HalfBitsToFloat): normals by exponent re-bias, subnormals as
 * mantissa * 2^-24; exponent 31 is NOT special-cased, so f16 inf/NaN come out as finite
 * values 2^16 * (1 + m/1024). */
static float f16_vec_decode(uint16_t h)
{
    uint32_t u = h;
    uint32_t sign = (u & 0x8000u) << 16, exp = (u >> 10) & 0x1Fu, man = (u & 0x3FFu) << 13;
    if (exp == 0) {
        float sub = (float)(u & 0x3FFu) * 5.9604645e-8f;
        return u2f(f2u(sub) | sign);
    }
    return u2f(sign | ((exp + 112u) << 23) | man);
}

/* DotKernels.cs:59-84 (F16), :106-128 (BF16), SimdMath.cs:34-53 (F32): 8 lane sums over
 * k = 8c + L, HSum, then a sequential tail (tail halves decoded by Dtypes.F16ToFloat). */
static float dot_fp(int fmt, const uint8_t* w, const float* x, int cols)
{
    const uint16_t* s = (const uint16_t*)w;
    if (fmt == 0) return qro_dot_f32((const float*)w, x, cols);
    if (cols >= 8) {
        float lanes[8] = {0};
        int i = 0;
        for (; i + 8 <= cols; i += 8)
            for (int j = 0; j < 8; j++) {
                float wv = fmt == 1 ? f16_vec_decode(s[i + j]) : qro_bf16_to_f32(s[i + j]);
                float p = wv * x[i + j];
                lanes[j] = lanes[j] + p;
            }
        float sum = hsum8(lanes);
        for (; i < cols; i++) {
            float wv = fmt == 1 ? qro_f16_to_f32(s[i]) : qro_bf16_to_f32(s[i]);
            float p = wv * x[i];
            sum = sum + p;
        }
        return sum;
    }
    float ss = 0.0f;
    for (int i = 0; i < cols; i++) {
        float wv = fmt == 1 ? qro_f16_to_f32(s[i]) : qro_bf16_to_f32(s[i]);
        float p = wv * x[i];
        ss = ss + p;
    }
    return ss;
}

/* DotKernels.cs:134-178: per block, lane L of accQ takes lo[L]x[L], lo[8+L]x[8+L],
 * hi[L]x[16+L], hi[8+L]x[24+L]; accX the same x's; sum += d*dotQ - 8*d*sumX. */
static float dot_q4_0(const uint8_t* w, const float* x, int cols)
{
    float sum = 0.0f;
    for (int b = 0; b < cols / 32; b++, w += 20, x += 32) {
        float d = qro_f16_to_f32(le16(w));
        float aq[8], ax[8];
        for (int L = 0; L < 8; L++) {
            float q0 = (float)(w[2 + L] & 0xF), q1 = (float)(w[2 + 8 + L] & 0xF);
            float q2 = (float)(w[2 + L] >> 4), q3 = (float)(w[2 + 8 + L] >> 4);
            float a = 0.0f, s = 0.0f, p;
            p = q0 * x[L]; a = a + p;
            p = q1 * x[8 + L]; a = a + p;
            p = q2 * x[16 + L]; a = a + p;
            p = q3 * x[24 + L]; a = a + p;
            s = s + x[L]; s = s + x[8 + L]; s = s + x[16 + L]; s = s + x[24 + L];
            aq[L] = a;
            ax[L] = s;
        }
        float dotq = hsum8(aq), sumx = hsum8(ax);
        float t1 = d * dotq, d8 = 8.0f * d, t2 = d8 * sumx, e = t1 - t2;
        sum = sum + e;
    }
    return sum;
}

/* DotKernels.cs:183-230 (DotQ8_0, DotI8Bytes): lane L takes q[L], q[8+L], q[16+L], q[24+L];
 * HSum; sum += d * dot. */
static float dot_q8_0(const uint8_t* w, const float* x, int cols)
{
    float sum = 0.0f;
    for (int b = 0; b < cols / 32; b++, w += 34, x += 32) {
        float d = qro_f16_to_f32(le16(w));
        float acc[8];
        for (int L = 0; L < 8; L++) {
            float a = 0.0f;
            for (int k = 0; k < 4; k++) {
                float p = (float)(int8_t)w[2 + 8 * k + L] * x[8 * k + L];
                a = a + p;
            }
            acc[L] = a;
        }
        float dot = hsum8(acc), e = d * dot;
        sum = sum + e;
    }
    return sum;
}

/* DotKernels.cs:361-373 (VecDot16): lane L = q[L]x[L] + q[8+L]x[8+L] (no leading zero), HSum. */
static float vecdot16(const float* q, const float* x)
{
    float acc[8];
    for (int L = 0; L < 8; L++) {
        float p0 = q[L] * x[L], p1 = q[8 + L] * x[8 + L];
        acc[L] = p0 + p1;
    }
    return hsum8(acc);
}

/* DotKernels.cs:264-270 (SubSum): sequential. */
static float subsum(const float* x, int n)
{
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + x[i];
    return s;
}

/* DotKernels.cs:322-358: per 64-weight group j, even sub-block (low nibbles of the 32
 * bytes) then odd (high nibbles): sum += a*(VecDot16 + VecDot16) - mm*SubSum(32). */
static float dot_q4_k(const uint8_t* w, const float* x, int cols)
{
    float sum = 0.0f;
    for (int b = 0; b < cols / 256; b++, w += 144, x += 256) {
        float d = qro_f16_to_f32(le16(w)), dmin = qro_f16_to_f32(le16(w + 2));
        const uint8_t* q = w + 16;
        for (int j = 0; j < 4; j++, q += 32) {
            for (int odd = 0; odd < 2; odd++) {
                int sc, m;
                scale_min_k4(2 * j + odd, w + 4, &sc, &m);
                float a = d * (float)sc, mm = dmin * (float)m;
                float lo[16], hi[16];
                for (int i = 0; i < 16; i++) {
                    lo[i] = (float)(odd ? (q[i] >> 4) : (q[i] & 0xF));
                    hi[i] = (float)(odd ? (q[16 + i] >> 4) : (q[16 + i] & 0xF));
                }
                const float* xs = x + j * 64 + 32 * odd;
                float v1 = vecdot16(lo, xs), v2 = vecdot16(hi, xs + 16), v = v1 + v2;
                float t1 = a * v, t2 = mm * subsum(xs, 32), e = t1 - t2;
                sum = sum + e;
            }
        }
    }
    return sum;
}

/* DotKernels.cs:420-447: dot += (float)(sc*(q-32)) * x in (half, l, q1..q4) order; sum += d*dot. */
static float dot_q6_k(const uint8_t* w, const float* x, int cols)
{
    float sum = 0.0f;
    for (int b = 0; b < cols / 256; b++, w += 210, x += 256) {
        float d = qro_f16_to_f32(le16(w + 208));
        const uint8_t *ql = w, *qh = w + 128;
        const int8_t* sc = (const int8_t*)(w + 192);
        float dot = 0.0f;
        for (int n = 0; n < 256; n += 128) {
            int sb = 8 * (n / 128);
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (ql[n / 2 + l] & 0xF) | (((qh[n / 4 + l] >> 0) & 3) << 4);
                int q2 = (ql[n / 2 + l + 32] & 0xF) | (((qh[n / 4 + l] >> 2) & 3) << 4);
                int q3 = (ql[n / 2 + l] >> 4) | (((qh[n / 4 + l] >> 4) & 3) << 4);
                int q4 = (ql[n / 2 + l + 32] >> 4) | (((qh[n / 4 + l] >> 6) & 3) << 4);
                float p;
                p = (float)(sc[sb + is + 0] * (q1 - 32)) * x[n + l]; dot = dot + p;
                p = (float)(sc[sb + is + 2] * (q2 - 32)) * x[n + l + 32]; dot = dot + p;
                p = (float)(sc[sb + is + 4] * (q3 - 32)) * x[n + l + 64]; dot = dot + p;
                p = (float)(sc[sb + is + 6] * (q4 - 32)) * x[n + l + 96]; dot = dot + p;
            }
        }
        float e = d * dot;
        sum = sum + e;
    }
    return sum;
}

float qro_dot_row(int fmt, const uint8_t* w, const float* x, int cols)
{
    switch (fmt) {
    case 0: case 1: case 2: return dot_fp(fmt, w, x, cols);
    case 3: return dot_q4_0(w, x, cols);
    case 4: return dot_q8_0(w, x, cols);
    case 6: return dot_q4_k(w, x, cols);
    case 7: return dot_q6_k(w, x, cols);
    }
    return NAN;
}

int qro_matvec(int fmt, const uint8_t* w, long rows, int cols, const float* x, float* y)
{
    long rb = qro_row_bytes(fmt, cols);
    if (rb < 0) return -1;
    for (long r = 0; r < rows; r++) y[r] = qro_dot_row(fmt, w + r * rb, x, cols);
    return 0;
}
