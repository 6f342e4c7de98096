/*
 * qr_attn.h -- C ABI of the MI355X (gfx950) paged-KV attention library.
 *
 * This is the drop-in boundary for QuantRunner's attention path.  The C#
 * classes PagedKvCache and MlaLatentCache keep their public members and
 * forward here through P/Invoke; every entry point below names the reference
 * member it replaces (paths relative to src/QuantRunner.Core).
 *
 * Conventions
 *  - Every call returns an int status: QR_OK (0) or a negative QR_ERR_* code.
 *    qr_last_error() returns a thread-local message for the last failure.
 *    Invalid arguments are reported, never dereferenced.
 *  - Handles are not thread-safe (the reference classes are not either);
 *    callers serialise calls on one handle.
 *  - Host-pointer calls are synchronous: on return the output is written and
 *    the inputs may be reused, like the reference's blocking methods.
 *  - *_dev calls take device pointers and a hipStream_t (passed as void*,
 *    NULL = the null stream) and return without synchronising.
 *  - A page holds QR_PAGE_TOKENS tokens.  Pages are allocated on first
 *    append of any of their positions and are zero-filled when allocated.
 *    Reset/Truncate keep pages (PagedKvCache.cs:72-76).
 *  - 16-bit data crosses the boundary as raw IEEE bit patterns (uint16_t).
 *    float -> fp16 conversion follows Dtypes.FloatToF16 (Dtypes.cs:100-126:
 *    ties away from zero in the normal range), float -> bf16 follows
 *    Dtypes.FloatToBf16 (round to nearest even, :132-139); 16-bit -> float
 *    is exact.
 */
#ifndef QR_ATTN_H
#define QR_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QR_ATTN_ABI_VERSION 1
#define QR_PAGE_TOKENS 256 /* PagedKvCache.PageTokens, PagedKvCache.cs:14 */

/* element types of caches and inputs */
enum {
    QR_DTYPE_F32 = 0,
    QR_DTYPE_F16 = 1,
    QR_DTYPE_BF16 = 2
};

/* weight-row formats: QuantFormat values, Dtypes.cs:6-26 (block specs :38-50).
 * The F32/F16/BF16 codes coincide with QR_DTYPE_*. */
enum {
    QR_FMT_F32 = 0,  /* 4 B / weight                                     */
    QR_FMT_F16 = 1,  /* 2 B / weight                                     */
    QR_FMT_BF16 = 2, /* 2 B / weight                                     */
    QR_FMT_Q4_0 = 3, /* 32 weights / 20 B: f16 d, 16 nibble bytes, 2 pad */
    QR_FMT_Q8_0 = 4, /* 32 weights / 34 B: f16 d, 32 int8                */
    QR_FMT_Q4_K = 6, /* 256 weights / 144 B                              */
    QR_FMT_Q6_K = 7  /* 256 weights / 210 B                              */
};

/* status codes */
enum {
    QR_OK = 0,
    QR_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad shape, dtype, layer or sequence id   */
    QR_ERR_OUT_OF_RANGE = -2,     /* pos >= max_seq, or a row longer than kv_dim           */
    QR_ERR_OUT_OF_MEMORY = -3,    /* device or host allocation failed                      */
    QR_ERR_HIP = -4,              /* a HIP runtime call failed (message has the HIP error) */
    QR_ERR_NOT_RESIDENT = -5      /* attention over a position whose page was never appended */
};

typedef struct qr_kv qr_kv;   /* PagedKvCache  */
typedef struct qr_mla qr_mla; /* MlaLatentCache */
typedef struct qr_weight qr_weight; /* one HBM-resident weight tensor (a ModelStore view) */

/* ---- library ---------------------------------------------------------- */
int qr_abi_version(void);
/* Thread-local message of the last failed call on this thread ("" if none). */
const char* qr_last_error(void);
/* Static name of a status code, e.g. "QR_ERR_OUT_OF_RANGE". */
const char* qr_status_name(int status);

/* ---- PagedKvCache ------------------------------------------------------ */

/* ctor PagedKvCache(layers, heads, kvHeads, headDim, maxSeq), PagedKvCache.cs:29-37.
 * kv_dtype: QR_DTYPE_F32 (the reference's page type, PagedKvCache.cs:17-18),
 * F16 or BF16.  max_batch: number of independent sequences (seq_id 0..max_batch-1),
 * each with its own page table; 1 reproduces the reference.  head_dim: any size from
 * 1 to 512 (the reference takes any).  16-bit caches with head_dim 64 or 128 decode on
 * MFMA tiles; multiples of 8 from 16 to 256 on the streaming kernel; every other size on
 * a scalar generic kernel (correct, not tuned: no model uses such sizes). */
int qr_kv_create(qr_kv** out, int layers, int heads, int kv_heads, int head_dim, int max_seq,
                 int kv_dtype, int max_batch);
int qr_kv_destroy(qr_kv* kv);

/* Pre-sizes the device page pool to hold at least `pages` pages so that later
 * appends do not grow it.  No reference counterpart (the reference allocates
 * per page from the managed heap). */
int qr_kv_reserve(qr_kv* kv, int pages);

/* Append(layer, pos, k, v), PagedKvCache.cs:62-69.  k/v are host fp32 rows of
 * k_len/v_len floats.  A row longer than kv_dim is an error (the reference's
 * Span.CopyTo throws); a shorter one overwrites only its first elements, as
 * Span.CopyTo does.  SeqLen(seq) = max(SeqLen, pos+1). */
int qr_kv_append(qr_kv* kv, int seq_id, int layer, int pos, const float* k, int k_len,
                 const float* v, int v_len);

/* Bulk Append of n consecutive positions pos0..pos0+n-1: k/v are host rows
 * [n][kv_dim] of src_dtype, converted to the cache dtype.  Equivalent to n
 * Append calls. */
int qr_kv_append_range(qr_kv* kv, int seq_id, int layer, int pos0, int n, const void* k,
                       const void* v, int src_dtype);
/* Same with device-resident rows, enqueued on `stream`. */
int qr_kv_append_range_dev(qr_kv* kv, int seq_id, int layer, int pos0, int n, const void* k_dev,
                           const void* v_dev, int src_dtype, void* stream);

/* Replaces the RoPE + Append step of StreamingEngine.Forward
 * (StreamingEngine.cs:245-248; TransformerOps.BuildCosSinInto / Rope, TransformerOps.cs:56-88;
 * PagedKvCache.Append, PagedKvCache.cs:62-69) for one position: the kv_dim-float k row
 * and the heads*head_dim q row are rotated in place in the reference's rotate-half
 * convention with cos/sin of pos * theta^(-2i/head_dim); the rotated k and the v row
 * are appended at pos, and the rotated q is written back to `q` (the reference rotates
 * pq in place before Attention).  k and v must be full kv_dim rows. */
int qr_kv_append_rope(qr_kv* kv, int seq_id, int layer, int pos, float* q, const float* k,
                      const float* v, float theta);
/* Same for n consecutive positions pos0..pos0+n-1 with device rows: q_dev
 * [n][heads*head_dim] (rotated in place; may be null), k_dev and v_dev [n][kv_dim] fp32,
 * each 16-byte aligned; enqueued on `stream`. */
int qr_kv_append_rope_dev(qr_kv* kv, int seq_id, int layer, int pos0, int n, float* q_dev,
                          const float* k_dev, const float* v_dev, float theta, void* stream);
/* Same for ONE position whose index is read on the device from *pos_dev (the Ensure +
 * Append of StreamingEngine.cs:245-248 with PagedKvCache.Ensure, PagedKvCache.cs:41-60,
 * done on the GPU): the pages up to the position are claimed from the pool by a device
 * counter and SeqLen's device copy grows to pos + 1, so a decode step built from this
 * call and qr_kv_attention_step_dev can be captured in a HIP graph and replayed at
 * advancing positions.  The pool cannot grow inside a capture: reserve enough pages
 * (qr_kv_reserve) before capturing, and make the cache's first device-side call outside
 * capture.  A full pool or a position outside [0, max_seq) skips the append and is
 * reported by the next host-side call on the cache (which waits for the device and
 * reads the page accounting back; QR_ERR_OUT_OF_MEMORY / QR_ERR_OUT_OF_RANGE).  Calls
 * on one cache must be ordered by the caller (one stream, or synchronised). */
int qr_kv_append_rope_step_dev(qr_kv* kv, int seq_id, int layer, const int* pos_dev, float* q_dev,
                               const float* k_dev, const float* v_dev, float theta, void* stream);
/* Same for the nq consecutive positions *pos0_dev .. *pos0_dev + nq - 1 of a chunk
 * (prompt chunk or draft tokens, StreamingEngine.cs:831-836 / SpeculativeRunner.cs:85-93
 * append each of them in turn): q_dev [nq][heads*head_dim], k_dev/v_dev
 * [nq][kv_heads*head_dim].  The pages up to the last position are claimed; positions
 * reaching past max_seq skip the append and are reported as above. */
int qr_kv_append_rope_chunk_step_dev(qr_kv* kv, int seq_id, int layer, int nq, const int* pos0_dev,
                                     float* q_dev, const float* k_dev, const float* v_dev, float theta,
                                     void* stream);

/* Attention(layer, pos, q, attn, scale), PagedKvCache.cs:83-136:
 * attn[h*D:(h+1)*D] = softmax(q_h . K[0..pos, kvh(h)] * scale) . V[0..pos, kvh(h)],
 * kvh(h) = h*kv_heads/heads.  q and attn are host fp32 [heads*head_dim]. */
int qr_kv_attention(qr_kv* kv, int seq_id, int layer, int pos, const float* q, float* attn,
                    float scale);

/* Attention (PagedKvCache.cs:83-136) for n <= 64 entries whose positions are read on
 * the device, entry i over sequence seq_ids[i] at position pos_dev[i] (device int32
 * array): the companion of qr_kv_append_rope_step_dev for captured decode steps.  The
 * split count is planned for max_seq and each entry's positions spread over it on the
 * device; the split workspace can only grow outside a capture, so make one call before
 * capturing.  Positions never appended read undefined values, as in the reference. */
int qr_kv_attention_step_dev(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos_dev,
                             const float* q_dev, float* attn_dev, float scale, void* stream);

/* n independent decode queries, entry i over sequence seq_ids[i] at position
 * pos[i]; q/attn are host fp32 [n][heads*head_dim].  Equivalent to n
 * qr_kv_attention calls. */
int qr_kv_attention_batch(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos,
                          const float* q, float* attn, float scale);
/* Same with device q/attn, enqueued on `stream`.  seq_ids/pos stay host arrays. */
int qr_kv_attention_dev(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos,
                        const float* q_dev, float* attn_dev, float scale, void* stream);

/* No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same as qr_kv_attention_dev, but the split partials live in a
 * fixed 8 MiB device array of the library (one per GPU, held until the process
 * ends) instead of the handle's workspace, which grows with hipMalloc; nothing is
 * allocated, on the host or the device.  The array's first 64 KiB hold the split
 * merge's arrival counters (zero between calls), the rest the partials.  At most 64
 * entries per call; a call whose split partials (entries x heads x splits x
 * (head_dim x 4 + 8) bytes) exceed 8 MiB - 64 KiB returns QR_ERR_OUT_OF_RANGE.  Every call on a GPU shares that GPU's array,
 * whatever the handle: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller. */
int qr_kv_attention_dev_noalloc(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos,
                                const float* q_dev, float* attn_dev, float scale, void* stream);

/* Causal multi-query attention over one sequence: query i sits at position
 * pos0+i and attends positions 0..pos0+i.  This is what nq sequential
 * Attention calls with interleaved appends compute (chunked prompt
 * processing, StreamingEngine.cs:831-836; speculative verify,
 * SpeculativeRunner.cs:85-93).  Positions pos0..pos0+nq-1 must already be
 * appended.  q: host [nq][heads*head_dim] in q_dtype; attn: host fp32. */
int qr_kv_attention_chunk(qr_kv* kv, int seq_id, int layer, int pos0, int nq, const void* q,
                          int q_dtype, float* attn, float scale);
int qr_kv_attention_chunk_dev(qr_kv* kv, int seq_id, int layer, int pos0, int nq,
                              const void* q_dev, int q_dtype, float* attn_dev, float scale,
                              void* stream);
/* Same with the position of query 0 read on the device from *pos0_dev (clamped to
 * [0, max_seq - nq]): the companion of qr_kv_append_rope_chunk_step_dev for captured
 * prefill / verify steps.  The split count is planned for max_seq and the keys of the
 * chunk spread over it on the device; the workspace grows only outside a capture (make
 * one call before capturing).  Caches without the MFMA chunk path (fp32, or head sizes
 * other than 64 / 128) take fp32 queries and at most 64 of them. */
int qr_kv_attention_chunk_step_dev(qr_kv* kv, int seq_id, int layer, int nq, const int* pos0_dev,
                                   const void* q_dev, int q_dtype, float* attn_dev, float scale,
                                   void* stream);

/* Benchmark instrumentation, no reference counterpart: when `event` (a
 * hipEvent_t) is not NULL, every later attention call records it on its
 * stream right after the split-K kernel and before the combine kernel, so a
 * caller can time the split-K kernel alone (a decode split-K kernel that merges
 * its own splits launches no combine kernel).  NULL turns it off. */
int qr_kv_set_split_event(qr_kv* kv, void* event);

/* Introspection, no reference counterpart: the split-K plan a decode call with
 * these entries would take (as qr_kv_attention_batch / _dev, first 64 entries):
 * tokens per split (a multiple of 256) and the number of splits of the longest
 * entry (1: the split kernel writes the output, no merge; more: the last split of
 * each kv head to finish merges them inside the split kernel when all splits run
 * in one pass of the GPU, else a merge kernel follows).  Validates like the
 * attention call; launches nothing. */
int qr_kv_decode_plan(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos, int* split_tokens,
                      int* splits);

/* Reset(), PagedKvCache.cs:72 (seq_id < 0 resets every sequence). */
int qr_kv_reset(qr_kv* kv, int seq_id);
/* Truncate(len), PagedKvCache.cs:76: SeqLen = min(SeqLen, len). */
int qr_kv_truncate(qr_kv* kv, int seq_id, int len);
/* SeqLen, PagedKvCache.cs:26. */
int qr_kv_seq_len(const qr_kv* kv, int seq_id, int* out);
/* BytesUsed, PagedKvCache.cs:27,56: pages x 256 x kv_dim x elem_bytes x 2 summed over
 * layers and sequences (elem_bytes 4 for f32, matching the reference; 2 for 16-bit). */
int qr_kv_bytes_used(const qr_kv* kv, long long* out);
/* BytesPerToken, PagedKvCache.cs:39: kv_dim x elem_bytes x 2 x layers. */
int qr_kv_bytes_per_token(const qr_kv* kv, long long* out);
/* Copies rows pos0..pos0+n-1 of one layer back to the host as cache-dtype
 * rows [n][kv_dim] (debug copy-out; positions must be resident). */
int qr_kv_read(qr_kv* kv, int seq_id, int layer, int pos0, int n, void* k_out, void* v_out);

/* ---- MlaLatentCache ---------------------------------------------------- */

/* ctor MlaLatentCache(layers, latentDim, maxSeq), MlaLatentCache.cs:22-27, with the
 * latent split given up front: latentDim = kv_lora + rope (StreamingEngine.cs:96).
 * dtype: F32, F16 or BF16.  1 <= kv_lora <= 1024, 0 <= rope <= 256.  16-bit caches
 * with kv_lora 512 and rope 0 or 64 run on MFMA tiles whose operands stay in the
 * cache's 16-bit type (any finite latent value); every other shape runs a generic
 * fp32 kernel. */
int qr_mla_create(qr_mla** out, int layers, int kv_lora, int rope, int max_seq, int dtype);
/* ctor MlaLatentCache(layers, latentDim, maxSeq) exactly as the reference takes it
 * (MlaLatentCache.cs:22; StreamingEngine.cs:96-97 passes kv_lora + rope): storage
 * needs the row width only.  The cache knows no kv_lora / rope split (the reference's
 * split lives in MlaLayer, StreamingEngine.cs:531-568), so attention calls return
 * QR_ERR_INVALID_ARGUMENT until qr_mla_set_rope fixes it.  latentDim <= 1280. */
int qr_mla_create_latent(qr_mla** out, int layers, int latent_dim, int max_seq, int dtype);
/* No reference counterpart: the rope width of the latent rows (kv_lora = latentDim -
 * rope), as MlaLayer knows it (Config.QkRopeHeadDim); may be set again at any time. */
int qr_mla_set_rope(qr_mla* m, int rope);
/* MaxSeq, MlaLatentCache.cs:65. */
int qr_mla_max_seq(const qr_mla* m, int* out);
int qr_mla_destroy(qr_mla* mla);
int qr_mla_reserve(qr_mla* mla, int pages);
/* Append(layer, pos, latent), MlaLatentCache.cs:45-51 (row of `len` floats <= latentDim). */
int qr_mla_append(qr_mla* mla, int layer, int pos, const float* latent, int len);
/* Bulk Append of rows [n][latentDim] in src_dtype. */
int qr_mla_append_range(qr_mla* mla, int layer, int pos0, int n, const void* rows, int src_dtype);
int qr_mla_append_range_dev(qr_mla* mla, int layer, int pos0, int n, const void* rows_dev,
                            int src_dtype, void* stream);
/* Absorbed attention against the latent cache, StreamingEngine.cs:531-568:
 *   s_t = (q_tilde_h . c_t[0:kv_lora] + q_rope_h . c_t[kv_lora:]) * scale
 *   u_h = sum_t softmax(s)_t * c_t[0:kv_lora]
 * for t = 0..pos.  q_tilde [heads][kv_lora], q_rope [heads][rope], u [heads][kv_lora],
 * all host fp32.  The q-absorb (:517-529) and W_UV (:569-576) projections stay
 * with the caller. */
int qr_mla_attention(qr_mla* mla, int layer, int pos, int heads, const float* q_tilde,
                     const float* q_rope, float scale, float* u);
int qr_mla_attention_dev(qr_mla* mla, int layer, int pos, int heads, const float* q_tilde_dev,
                         const float* q_rope_dev, float scale, float* u_dev, void* stream);
/* The whole absorbed block of MlaLayer after cache.Append, StreamingEngine.cs:508-577:
 *   q~_h = sum_{j<nope} q_h[j] * W_kvb[h*(nope+vdim)+j]          (:517-529)
 *   u_h  = absorbed attention over positions 0..pos, scale 1/sqrt(nope+rope) (:511, :531-568)
 *   out_h[j] = DotF32(W_kvb[h*(nope+vdim)+nope+j], u_h)         (:569-576)
 * q [heads][nope+rope] fp32 (rope part already rotated, :499-501), out [heads][vdim].
 * kvb: [heads*(nope+vdim)][kv_lora] weights (qr_weight_create), decoded on the fly
 * exactly as BlockDequantizer.Dequantize; kv_lora a multiple of 8 and of the format's
 * block.  The projections reproduce the reference's fp32 operation order bit for bit. */
int qr_mla_attend_absorbed(qr_mla* mla, int layer, int pos, int heads, int nope, int vdim,
                           const float* q, const qr_weight* kvb, float* out);
/* Same on device buffers: kvb_dev 16-byte aligned, q_dev/out_dev 8-byte aligned. */
int qr_mla_attend_absorbed_dev(qr_mla* mla, int layer, int pos, int heads, int nope, int vdim,
                               const float* q_dev, const void* kvb_dev, int kvb_format,
                               float* out_dev, void* stream);
/* Device-position forms, no reference counterpart (for captured decode, prefill-chunk
 * and verify steps, as qr_kv_append_rope_step_dev / qr_kv_attention_step_dev): the n
 * latent rows rows_dev [n][latentDim] go to positions *pos0_dev .. *pos0_dev + n - 1,
 * their pages claimed on the device (Append, MlaLatentCache.cs:45-51); the attention and
 * the absorbed block run at position *pos_dev, read on the device (the split count is
 * planned for max_seq and the sequence spreads over it).  Reserve pages (qr_mla_reserve)
 * before capturing and make the cache's first device-position call outside capture; a
 * full pool or positions outside [0, max_seq) skip the append and are reported by the
 * next host-side call (QR_ERR_OUT_OF_MEMORY / QR_ERR_OUT_OF_RANGE). */
int qr_mla_append_step_dev(qr_mla* mla, int layer, int n, const int* pos0_dev, const void* rows_dev,
                           int src_dtype, void* stream);
int qr_mla_attention_step_dev(qr_mla* mla, int layer, const int* pos_dev, int heads,
                              const float* q_tilde_dev, const float* q_rope_dev, float scale,
                              float* u_dev, void* stream);
int qr_mla_attend_absorbed_step_dev(qr_mla* mla, int layer, const int* pos_dev, int heads, int nope,
                                    int vdim, const float* q_dev, const void* kvb_dev, int kvb_format,
                                    float* out_dev, void* stream);
int qr_mla_reset(qr_mla* mla);                    /* MlaLatentCache.cs:53 */
int qr_mla_truncate(qr_mla* mla, int len);        /* MlaLatentCache.cs:57 */
int qr_mla_seq_len(const qr_mla* mla, int* out);  /* MlaLatentCache.cs:19 */
int qr_mla_bytes_used(const qr_mla* mla, long long* out); /* MlaLatentCache.cs:20,40 */
int qr_mla_page_count(const qr_mla* mla, int layer, int* out); /* MlaLatentCache.cs:60 */
/* Page(layer, page), MlaLatentCache.cs:63: copies one page out as fp32
 * [256][latentDim] (16-bit caches decoded exactly). */
int qr_mla_read_page(qr_mla* mla, int layer, int page, float* out);

/* ---- weights and MLA projections -------------------------------------- */

/* Bytes of one row of `cols` weights (Dtypes.TensorBytes, Dtypes.cs:38-60). */
int qr_weight_row_bytes(int format, int cols, long long* out);
/* Uploads one weight tensor (rows x cols, rows back to back in `format`) into HBM on
 * the current device: the ModelStore view a layer reads (ModelStore.cs, RowPtr/RowBytes). */
int qr_weight_create(qr_weight** out, int format, long long rows, int cols, const void* host_bytes);
int qr_weight_destroy(qr_weight* w);
int qr_weight_data(const qr_weight* w, const void** dev_ptr);
/* q-absorb, StreamingEngine.cs:517-529, for nq query rows:
 *   q_tilde[b][h][k] = (((0 + q[b][h][0]*W[h*(nope+vdim)+0][k]) + q[b][h][1]*W[..+1][k]) + ...)
 * rows dequantized as BlockDequantizer.Dequantize (:524-526).  q_dev [nq][heads][nope+rope],
 * q_tilde_dev [nq][heads][kv_lora] (8-byte aligned), kvb_dev 16-byte aligned. */
int qr_mla_q_absorb_dev(const void* kvb_dev, int kvb_format, int heads, int nope, int rope, int vdim,
                        int kv_lora, int nq, const float* q_dev, float* q_tilde_dev, void* stream);
/* W_UV, StreamingEngine.cs:569-576: out[b][h][j] = DotF32(W[h*(nope+vdim)+nope+j], u[b][h])
 * with SimdMath.DotF32's lane order.  u_dev [nq][heads][kv_lora] (8-byte aligned),
 * out_dev [nq][heads][vdim]. */
int qr_mla_wuv_dev(const void* kvb_dev, int kvb_format, int heads, int nope, int vdim, int kv_lora,
                   int nq, const float* u_dev, float* out_dev, void* stream);
/* MatVec / MatVecParallel, DotKernels.cs:599-633: y[b][r] = DotRow(W row r, x[b]) for nq input
 * vectors, each row in its format's own fused dequant + dot order (DotKernels.cs:24-447), so
 * every y[r] equals the reference's bit for bit.  w_dev [rows][row bytes] 16-byte aligned;
 * x_dev [nq][cols] 16-byte aligned; y_dev [nq][rows].  cols: whole blocks of the format,
 * and a multiple of 8 for F32/F16/BF16. */
int qr_matvec_dev(const void* w_dev, int format, long long rows, int cols, int nq, const float* x_dev,
                  float* y_dev, void* stream);
/* n <= 4 MatVecs that read the same x -- the projections of one activation vector, as
 * StreamingEngine.cs:240-242 (wq, wk, wv of the normed x) and :605-606 (gate and up) call
 * MatVecParallel on them one after another -- with one launch for F32/F16/BF16 rows (the
 * other formats run one launch per matrix).  Same format and cols for every matrix; matrix m
 * has rows[m] rows at w_devs[m] (16-byte aligned) and writes y_devs[m] [nq][rows[m]].  Every
 * y equals qr_matvec_dev's for that matrix, bit for bit.  No counterpart in the reference:
 * for callers that run a layer's projections on the GPU. */
int qr_matvec_group_dev(int n, const void* const* w_devs, const long long* rows, int format, int cols, int nq,
                        const float* x_dev, float* const* y_devs, void* stream);
/* Same with host vectors against an uploaded weight (synchronous; not thread-safe per weight). */
int qr_matvec(const qr_weight* w, int nq, const float* x, float* y);

/* ---------------------------------------------------------------- .qw weight files in HBM
 * A qr_model is one opened .qw file (ModelStore) plus its layer prefetch pipeline
 * (PrefetchPipeline).  The file stays open; tensors are read with positional reads.  Device
 * memory is taken on the device current at the first Begin / Acquire / make_resident call.
 * A handle is used from one host thread at a time. */
typedef struct qr_model qr_model;
/* ModelStore.Open, ModelStore.cs:85-126: "QWR1", int32 header length, JSON header
 * {config, tensors[{name, dims, format, offset, size}], data_offset?}; data starts at the
 * 64-byte-aligned data_offset (or header end).  Host only: no device call. */
int qr_model_open(qr_model** out, const char* path);
/* ModelStore.Dispose + PrefetchPipeline.Dispose (ModelStore.cs:128-132, PrefetchPipeline.cs:179-189):
 * waits for pending reads, uploads and the work that acquired a slot, then frees everything. */
int qr_model_close(qr_model* m);
/* ModelStore.Tensors (ModelStore.cs:69): count and names in header order. */
int qr_model_tensor_count(const qr_model* m, int* count);
int qr_model_tensor_name(const qr_model* m, int index, char* buf, int buf_len);
/* TensorView.Format / Dims / SizeBytes (ModelStore.cs:10-27) of ModelStore.Get(name) (:79-80). */
int qr_model_tensor_info(const qr_model* m, const char* name, int* format, int* ndims, long long* dims,
                         int dims_cap, long long* bytes);
/* TensorView.Bytes (ModelStore.cs:27): the tensor's bytes into host memory. */
int qr_model_read(const qr_model* m, const char* name, void* dst, long long dst_bytes);
/* new PrefetchPipeline(store, budgetBytes), PrefetchPipeline.cs:52-61: 0 disables staging. */
int qr_model_set_prefetch(qr_model* m, long long budget_bytes);
/* PrefetchPipeline.Begin, PrefetchPipeline.cs:64-75: starts staging layer `layer` (tensors named
 * "l<layer>.*" except those ending in "norm" or "router"; every tensor for a negative layer) into
 * HBM slot layer & 1.  The slot's next upload waits, on the GPU, for the work queued so far on
 * every stream that acquired the slot's previous layer: pointers of that layer are not valid
 * for work queued after this call. */
int qr_model_begin(qr_model* m, int layer);
/* PrefetchPipeline.Acquire, PrefetchPipeline.cs:82-97: device address of tensor `name` as layer
 * `layer` uses it.  Staged: `stream` waits on the GPU for the slot's upload.  Not staged (layer
 * never begun, over budget, read failed, norms and routers, pipeline off): the tensor is uploaded
 * once and kept, as the reference falls back to its mmap view. */
int qr_model_acquire(qr_model* m, const char* name, int layer, void* stream, const void** dev_ptr);
/* No counterpart in the reference (its compute is synchronous): marks the end of the work that
 * `stream` queued on layer `layer`'s staged tensors, so the slot's next upload can start as soon
 * as that work is done instead of waiting for everything queued before the next Begin.  Call it
 * after the layer's last launch on each stream that acquired it; without it, Begin fences. */
int qr_model_release(qr_model* m, int layer, void* stream);
/* PrefetchPipeline.WaitLayer, PrefetchPipeline.cs:100-109: waits for the layer's file read. */
int qr_model_wait_layer(qr_model* m, int layer);
/* No counterpart in the reference: uploads every tensor once into one HBM allocation, after
 * which Acquire serves all of them with no copy and no wait.  For models that fit in HBM. */
int qr_model_make_resident(qr_model* m);
/* PrefetchPipeline BytesStreamed / WaitTicks / ReadTicks / StagedLayers / SkippedLayers
 * (PrefetchPipeline.cs:40-48), times in milliseconds. */
int qr_model_stats(qr_model* m, long long* bytes_streamed, double* wait_ms, double* read_ms, int* staged_layers,
                   int* skipped_layers);

#ifdef __cplusplus
}
#endif
#endif /* QR_ATTN_H */
