// qr_mla.cpp -- C ABI of the paged MLA latent cache (MlaLatentCache, MlaLatentCache.cs:10-65)
// and of the absorbed attention over it (StreamingEngine.cs:531-568).
#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "qr_mla.hpp"
#include "qr_proj.hpp"
#include "qr_store.hpp"

using namespace qr;

struct qr_mla {
    int device = 0;
    int layers = 0, kv_lora = 0, rope = 0, latent = 0, max_seq = 0, dtype = 0;
    bool split_set = true;  // false until qr_mla_set_rope for caches made by qr_mla_create_latent
    PagedStore store;
    int seq_len = 0;
    hipStream_t stream = nullptr;
    DevBuf stage;
    DevBuf workspace;
    DevBuf proj;  // q_tilde, u and q_rope of the absorbed layer call
    bool device_steps = false;  // the device copy of the page accounting is in use
};

namespace {

int check_handle(const qr_mla* m) {
    if (!m) {
        set_error("null qr_mla handle");
        return QR_ERR_INVALID_ARGUMENT;
    }
    return QR_OK;
}

int check_layer(const qr_mla* m, int layer) {
    QR_CHECK_ARG(layer >= 0 && layer < m->layers, "layer %d outside [0, %d)", layer, m->layers);
    return QR_OK;
}

int check_pos(const qr_mla* m, int pos) {
    if (pos < 0 || pos >= m->max_seq) {
        set_error("position %d outside [0, max_seq=%d)", pos, m->max_seq);
        return QR_ERR_OUT_OF_RANGE;
    }
    return QR_OK;
}

int check_resident(const qr_mla* m, int layer, int pos) {
    if (!m->store.resident(0, layer, pos)) {
        set_error("position %d of layer %d was never appended (%d pages resident)", pos, layer,
                  m->store.pages_held(0, layer));
        return QR_ERR_NOT_RESIDENT;
    }
    return QR_OK;
}

// Host view of the page accounting and SeqLen, read back from the device after
// device-side appends (a no-op otherwise).  A device-pointer call enqueued under stream
// capture skips the read-back (it would wait for the device): its checks then use the
// host accounting, which never runs ahead of the device's.
bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

int sync_host(const qr_mla* cm, hipStream_t stream = nullptr, bool device_call = false) {
    qr_mla* m = const_cast<qr_mla*>(cm);
    if (!m->store.device_ahead()) return QR_OK;
    if (device_call && capturing(stream)) return QR_OK;
    DeviceGuard dg(m->device);
    std::vector<int> len{m->seq_len};
    const int st = m->store.pull(len);
    m->seq_len = len[0];
    return st;
}

// A call enqueued under stream capture leaves the addresses of the pool, the split
// workspace and the projection buffers in the graph: from then on the pool never moves
// (growing it is an error) and a buffer that grows keeps its old allocation alive for
// the graph's replays until the handle is destroyed.
void note_capture(qr_mla* m, hipStream_t stream) {
    if (!capturing(stream)) return;
    m->store.freeze();
    m->workspace.keep_retired();
    m->proj.keep_retired();
}

// Device copy of the accounting after host-side changes (once device-side appends are in use).
int sync_device(qr_mla* m, hipStream_t stream) {
    if (!m->device_steps) return QR_OK;
    return m->store.push(std::vector<int>{m->seq_len}, stream);
}

// SeqLen changed on the host (Reset / Truncate): the device copy follows before the call returns.
int sync_state(qr_mla* m) {
    if (!m->device_steps) return QR_OK;
    DeviceGuard dg(m->device);
    QR_TRY(sync_device(m, m->stream));
    QR_HIP(hipStreamSynchronize(m->stream));
    return QR_OK;
}

// A buffer that may only grow outside stream capture.
int ensure_outside_capture(DevBuf& b, size_t bytes, hipStream_t stream) {
    if (bytes <= b.size()) return QR_OK;
    QR_CHECK_ARG(!capturing(stream), "a buffer must grow to %zu bytes: make one call outside capture first", bytes);
    return b.ensure(bytes);
}

int append_dev(qr_mla* m, int layer, int pos0, int n, const void* rows, int len, int src_dtype,
               hipStream_t stream) {
    QR_TRY(m->store.ensure(0, layer, pos0 + n, stream));
    AppendArgs a{};
    a.pool = m->store.pool();
    a.page_table = m->store.page_table_dev() + m->store.pt_offset(0, layer);
    a.geom = m->store.geom();
    a.dtype = m->dtype;
    a.src[0] = rows;
    a.src[1] = nullptr;
    a.row_len[0] = len;
    a.row_len[1] = 0;
    a.src_stride = m->latent;
    a.src_dtype = src_dtype;
    a.pos0 = pos0;
    a.n = n;
    QR_HIP(launch_append(a, stream));
    m->seq_len = std::max(m->seq_len, pos0 + n);  // MlaLatentCache.cs:50
    return sync_device(m, stream);
}

// pos_dev set: the position is read on the device, pos is ignored and the plan is made
// for max_seq.
int attention_dev(qr_mla* m, int layer, int pos, const int* pos_dev, int heads, const float* qt,
                  const float* qr_, float scale, float* u, hipStream_t stream) {
    MlaArgs a{};
    a.pool = m->store.pool();
    a.page_table = m->store.page_table_dev() + m->store.pt_offset(0, layer);
    a.dtype = m->dtype;
    a.kv_lora = m->kv_lora;
    a.rope = m->rope;
    a.heads = heads;
    a.seq_len = pos_dev ? m->max_seq : pos + 1;
    a.pos_dev = pos_dev;
    a.q_tilde = qt;
    a.q_rope = qr_;
    a.u = u;
    a.scale = scale;
    const MlaPlan plan = plan_mla(a);
    QR_TRY(ensure_outside_capture(m->workspace, std::max<size_t>(plan.workspace_bytes, 256), stream));
    QR_HIP(launch_mla(a, plan, m->workspace.get(), stream));
    return QR_OK;
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// StreamingEngine.cs:508-577 after cache.Append: q-absorb, absorbed attention, W_UV.
int attend_absorbed_dev(qr_mla* m, int layer, int pos, const int* pos_dev, int heads, int nope, int vdim,
                        const float* q, const void* kvb, int fmt, float* out, hipStream_t stream) {
    MlaProjArgs a{};
    QR_TRY(mla_proj_prepare(a, kvb, fmt, heads, nope, m->rope, vdim, m->kv_lora));
    const size_t qt_bytes = align256(static_cast<size_t>(heads) * m->kv_lora * 4);
    const size_t qr_bytes = align256(static_cast<size_t>(heads) * std::max(m->rope, 1) * 4);
    QR_TRY(ensure_outside_capture(m->proj, 2 * qt_bytes + qr_bytes, stream));
    char* base = static_cast<char*>(m->proj.get());
    float* qt = reinterpret_cast<float*>(base);
    float* u = reinterpret_cast<float*>(base + qt_bytes);
    float* qr_ = reinterpret_cast<float*>(base + 2 * qt_bytes);
    a.nq = 1;
    a.in = q;
    a.out = qt;
    a.q_rope = m->rope > 0 ? qr_ : nullptr;
    QR_HIP(launch_mla_absorb(a, stream));
    const float scale = 1.0f / std::sqrt(static_cast<float>(nope + m->rope));  // :511
    QR_TRY(attention_dev(m, layer, pos, pos_dev, heads, qt, qr_, scale, u, stream));
    a.in = u;
    a.out = out;
    a.q_rope = nullptr;
    QR_HIP(launch_mla_wuv(a, stream));
    return QR_OK;
}

int validate_attention(const qr_mla* m, int layer, int pos, int heads) {
    QR_CHECK_ARG(m->split_set, "the latent's kv_lora/rope split is not set (qr_mla_set_rope)");
    QR_TRY(check_layer(m, layer));
    QR_TRY(check_pos(m, pos));
    QR_TRY(check_resident(m, layer, pos));
    QR_CHECK_ARG(heads >= 1 && heads <= kMlaMaxHeads, "heads %d outside [1, %d]", heads, kMlaMaxHeads);
    return QR_OK;
}

}  // namespace

extern "C" {

int qr_mla_create_latent(qr_mla** out, int layers, int latent_dim, int max_seq, int dtype) {
    clear_error();
    QR_CHECK_ARG(out != nullptr, "null output handle pointer");
    *out = nullptr;
    QR_CHECK_ARG(latent_dim >= 1 && latent_dim <= kMlaMaxLora + kMlaMaxRope, "latent_dim %d outside [1, %d]",
                 latent_dim, kMlaMaxLora + kMlaMaxRope);
    // storage needs the row width only; the split is fixed by qr_mla_set_rope
    const int kv_lora = std::min(latent_dim, kMlaMaxLora);
    const int st = qr_mla_create(out, layers, kv_lora, latent_dim - kv_lora, max_seq, dtype);
    if (st == QR_OK) (*out)->split_set = false;
    return st;
}

int qr_mla_set_rope(qr_mla* m, int rope) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_CHECK_ARG(rope >= 0 && rope <= kMlaMaxRope && rope < m->latent && m->latent - rope <= kMlaMaxLora,
                 "rope %d does not split a latent of %d into kv_lora <= %d and rope <= %d", rope, m->latent,
                 kMlaMaxLora, kMlaMaxRope);
    m->rope = rope;
    m->kv_lora = m->latent - rope;
    m->split_set = true;
    return QR_OK;
}

int qr_mla_max_seq(const qr_mla* m, int* out) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_CHECK_ARG(out, "null output pointer");
    *out = m->max_seq;
    return QR_OK;
}

int qr_mla_create(qr_mla** out, int layers, int kv_lora, int rope, int max_seq, int dtype) {
    clear_error();
    QR_CHECK_ARG(out != nullptr, "null output handle pointer");
    *out = nullptr;
    QR_CHECK_ARG(layers >= 1, "layers must be >= 1 (got %d)", layers);
    QR_CHECK_ARG(kv_lora >= 1 && kv_lora <= kMlaMaxLora, "kv_lora %d outside [1, %d]", kv_lora, kMlaMaxLora);
    QR_CHECK_ARG(rope >= 0 && rope <= kMlaMaxRope, "rope %d outside [0, %d]", rope, kMlaMaxRope);
    QR_CHECK_ARG(max_seq >= 1, "max_seq must be >= 1 (got %d)", max_seq);
    QR_CHECK_ARG(dtype_valid(dtype), "unknown dtype %d", dtype);
    qr_mla* m = new (std::nothrow) qr_mla();
    if (!m) {
        set_error("host allocation of the handle failed");
        return QR_ERR_OUT_OF_MEMORY;
    }
    m->layers = layers;
    m->kv_lora = kv_lora;
    m->rope = rope;
    m->latent = kv_lora + rope;
    m->max_seq = max_seq;
    m->dtype = dtype;
    int st = QR_OK;
    if (hipGetDevice(&m->device) != hipSuccess) {
        set_error("no HIP device available");
        st = QR_ERR_HIP;
    }
    if (st == QR_OK) {
        PageGeom g{1, 1, m->latent};
        st = m->store.init(g, dtype, layers, 1, max_seq);
    }
    if (st == QR_OK && hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
        set_error("hipStreamCreateWithFlags failed");
        st = QR_ERR_HIP;
    }
    if (st != QR_OK) {
        if (m->stream) (void)hipStreamDestroy(m->stream);
        delete m;
        return st;
    }
    *out = m;
    return QR_OK;
}

int qr_mla_destroy(qr_mla* m) {
    clear_error();
    if (!m) return QR_OK;
    DeviceGuard dg(m->device);
    (void)hipStreamSynchronize(m->stream);
    (void)hipStreamDestroy(m->stream);
    delete m;
    return QR_OK;
}

int qr_mla_reserve(qr_mla* m, int pages) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    DeviceGuard dg(m->device);
    return m->store.reserve(pages);
}

int qr_mla_append(qr_mla* m, int layer, int pos, const float* latent, int len) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_TRY(check_layer(m, layer));
    QR_TRY(check_pos(m, pos));
    QR_CHECK_ARG(len >= 0 && (latent || len == 0), "null latent row");
    if (len > m->latent) {
        set_error("row of %d floats is longer than the latent width %d", len, m->latent);
        return QR_ERR_OUT_OF_RANGE;
    }
    DeviceGuard dg(m->device);
    QR_TRY(m->stage.ensure(static_cast<size_t>(m->latent) * 4));
    if (len) QR_HIP(hipMemcpyAsync(m->stage.get(), latent, len * 4, hipMemcpyHostToDevice, m->stream));
    QR_TRY(append_dev(m, layer, pos, 1, m->stage.get(), len, QR_DTYPE_F32, m->stream));
    QR_HIP(hipStreamSynchronize(m->stream));
    return QR_OK;
}

int qr_mla_append_range(qr_mla* m, int layer, int pos0, int n, const void* rows, int src_dtype) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(dtype_valid(src_dtype), "unknown source dtype %d", src_dtype);
    QR_CHECK_ARG(n >= 0 && (rows || n == 0), "null rows / negative count");
    if (n == 0) return QR_OK;
    QR_TRY(check_pos(m, pos0));
    QR_TRY(check_pos(m, pos0 + n - 1));
    DeviceGuard dg(m->device);
    const size_t bytes = static_cast<size_t>(n) * m->latent * dtype_size(src_dtype);
    QR_TRY(m->stage.ensure(bytes));
    QR_HIP(hipMemcpyAsync(m->stage.get(), rows, bytes, hipMemcpyHostToDevice, m->stream));
    QR_TRY(append_dev(m, layer, pos0, n, m->stage.get(), m->latent, src_dtype, m->stream));
    QR_HIP(hipStreamSynchronize(m->stream));
    return QR_OK;
}

int qr_mla_append_range_dev(qr_mla* m, int layer, int pos0, int n, const void* rows_dev, int src_dtype,
                            void* stream) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m, static_cast<hipStream_t>(stream), true));
    note_capture(m, static_cast<hipStream_t>(stream));
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(dtype_valid(src_dtype), "unknown source dtype %d", src_dtype);
    QR_CHECK_ARG(n >= 0 && (rows_dev || n == 0), "null rows / negative count");
    if (n == 0) return QR_OK;
    QR_TRY(check_pos(m, pos0));
    QR_TRY(check_pos(m, pos0 + n - 1));
    DeviceGuard dg(m->device);
    return append_dev(m, layer, pos0, n, rows_dev, m->latent, src_dtype, static_cast<hipStream_t>(stream));
}

int qr_mla_attention(qr_mla* m, int layer, int pos, int heads, const float* q_tilde, const float* q_rope,
                     float scale, float* u) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_CHECK_ARG(q_tilde && u && (q_rope || m->rope == 0), "null q_tilde/q_rope/u pointer");
    QR_TRY(validate_attention(m, layer, pos, heads));
    DeviceGuard dg(m->device);
    const size_t qt_bytes = static_cast<size_t>(heads) * m->kv_lora * 4;
    const size_t qr_bytes = static_cast<size_t>(heads) * m->rope * 4;
    QR_TRY(m->stage.ensure(2 * qt_bytes + qr_bytes + 512));
    char* st = static_cast<char*>(m->stage.get());
    float* dqt = reinterpret_cast<float*>(st);
    float* du = reinterpret_cast<float*>(st + qt_bytes);
    float* dqr = reinterpret_cast<float*>(st + 2 * qt_bytes);
    QR_HIP(hipMemcpyAsync(dqt, q_tilde, qt_bytes, hipMemcpyHostToDevice, m->stream));
    if (qr_bytes) QR_HIP(hipMemcpyAsync(dqr, q_rope, qr_bytes, hipMemcpyHostToDevice, m->stream));
    QR_TRY(attention_dev(m, layer, pos, nullptr, heads, dqt, dqr, scale, du, m->stream));
    QR_HIP(hipMemcpyAsync(u, du, qt_bytes, hipMemcpyDeviceToHost, m->stream));
    QR_HIP(hipStreamSynchronize(m->stream));
    return QR_OK;
}

int qr_mla_attention_dev(qr_mla* m, int layer, int pos, int heads, const float* q_tilde_dev,
                         const float* q_rope_dev, float scale, float* u_dev, void* stream) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m, static_cast<hipStream_t>(stream), true));
    note_capture(m, static_cast<hipStream_t>(stream));
    QR_CHECK_ARG(q_tilde_dev && u_dev && (q_rope_dev || m->rope == 0), "null q_tilde/q_rope/u pointer");
    QR_TRY(validate_attention(m, layer, pos, heads));
    DeviceGuard dg(m->device);
    return attention_dev(m, layer, pos, nullptr, heads, q_tilde_dev, q_rope_dev, scale, u_dev,
                         static_cast<hipStream_t>(stream));
}

int qr_mla_attend_absorbed(qr_mla* m, int layer, int pos, int heads, int nope, int vdim, const float* q,
                           const qr_weight* kvb, float* out) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_CHECK_ARG(q && out && kvb, "null q / kvb / out pointer");
    QR_TRY(validate_attention(m, layer, pos, heads));
    QR_CHECK_ARG(nope >= 1 && vdim >= 1, "bad nope %d / vdim %d", nope, vdim);
    QR_CHECK_ARG(kvb->rows == static_cast<long long>(heads) * (nope + vdim) && kvb->cols == m->kv_lora,
                 "kvb is %lld x %d, expected %lld x %d", kvb->rows, kvb->cols,
                 static_cast<long long>(heads) * (nope + vdim), m->kv_lora);
    QR_CHECK_ARG(kvb->device == m->device, "kvb lives on device %d, the cache on %d", kvb->device, m->device);
    DeviceGuard dg(m->device);
    const size_t q_bytes = static_cast<size_t>(heads) * (nope + m->rope) * 4;
    const size_t o_bytes = static_cast<size_t>(heads) * vdim * 4;
    QR_TRY(m->stage.ensure(align256(q_bytes) + o_bytes));
    char* st = static_cast<char*>(m->stage.get());
    float* dq = reinterpret_cast<float*>(st);
    float* dout = reinterpret_cast<float*>(st + align256(q_bytes));
    QR_HIP(hipMemcpyAsync(dq, q, q_bytes, hipMemcpyHostToDevice, m->stream));
    QR_TRY(attend_absorbed_dev(m, layer, pos, nullptr, heads, nope, vdim, dq, kvb->dev, kvb->format, dout, m->stream));
    QR_HIP(hipMemcpyAsync(out, dout, o_bytes, hipMemcpyDeviceToHost, m->stream));
    QR_HIP(hipStreamSynchronize(m->stream));
    return QR_OK;
}

int qr_mla_attend_absorbed_dev(qr_mla* m, int layer, int pos, int heads, int nope, int vdim, const float* q_dev,
                               const void* kvb_dev, int kvb_format, float* out_dev, void* stream) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m, static_cast<hipStream_t>(stream), true));
    note_capture(m, static_cast<hipStream_t>(stream));
    QR_CHECK_ARG(q_dev && out_dev, "null q / out pointer");
    QR_TRY(validate_attention(m, layer, pos, heads));
    DeviceGuard dg(m->device);
    return attend_absorbed_dev(m, layer, pos, nullptr, heads, nope, vdim, q_dev, kvb_dev, kvb_format, out_dev,
                               static_cast<hipStream_t>(stream));
}

int qr_mla_reset(qr_mla* m) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    m->seq_len = 0;
    return sync_state(m);
}

int qr_mla_truncate(qr_mla* m, int len) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    if (len < m->seq_len) m->seq_len = len;  // MlaLatentCache.cs:57
    return sync_state(m);
}

int qr_mla_seq_len(const qr_mla* m, int* out) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_CHECK_ARG(out, "null output pointer");
    *out = m->seq_len;
    return QR_OK;
}

int qr_mla_bytes_used(const qr_mla* m, long long* out) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_CHECK_ARG(out, "null output pointer");
    *out = m->store.bytes_used();
    return QR_OK;
}

int qr_mla_page_count(const qr_mla* m, int layer, int* out) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(out, "null output pointer");
    *out = m->store.pages_held(0, layer);
    return QR_OK;
}

int qr_mla_read_page(qr_mla* m, int layer, int page, float* out) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(sync_host(m));
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(out, "null output pointer");
    QR_CHECK_ARG(page >= 0 && page < m->store.pages_held(0, layer), "page %d outside [0, %d)", page,
                 m->store.pages_held(0, layer));
    DeviceGuard dg(m->device);
    const size_t bytes = static_cast<size_t>(kPageTokens) * m->latent * 4;
    QR_TRY(m->stage.ensure(bytes));
    GatherArgs g{};
    g.pool = m->store.pool();
    g.page_table = m->store.page_table_dev() + m->store.pt_offset(0, layer);
    g.geom = m->store.geom();
    g.dtype = m->dtype;
    g.dst[0] = m->stage.get();
    g.pos0 = page * kPageTokens;
    g.n = kPageTokens;
    g.to_f32 = 1;
    QR_HIP(launch_gather(g, m->stream));
    QR_HIP(hipMemcpyAsync(out, m->stage.get(), bytes, hipMemcpyDeviceToHost, m->stream));
    QR_HIP(hipStreamSynchronize(m->stream));
    return QR_OK;
}

int qr_mla_append_step_dev(qr_mla* m, int layer, int n, const int* pos0_dev, const void* rows_dev, int src_dtype,
                           void* stream) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(dtype_valid(src_dtype), "unknown source dtype %d", src_dtype);
    QR_CHECK_ARG(pos0_dev && rows_dev, "null pos/rows pointer");
    QR_CHECK_ARG(n >= 1 && n <= m->max_seq, "n %d outside [1, %d]", n, m->max_seq);
    DeviceGuard dg(m->device);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool cap = capturing(st);
    note_capture(m, st);
    if (!m->device_steps) {
        // first device-side append: the device copy starts from the host accounting
        QR_CHECK_ARG(!cap, "the first device-side append of a cache must run outside stream capture");
        QR_TRY(sync_host(m));
        m->device_steps = true;
        QR_TRY(m->store.push(std::vector<int>{m->seq_len}, st));
    }
    if (m->store.capacity() < 1) {
        QR_CHECK_ARG(!cap, "the page pool is empty: reserve pages before capturing device-side appends");
        QR_TRY(m->store.reserve(16));
    }
    PageClaimArgs c{};
    c.page_table = const_cast<int*>(m->store.page_table_dev()) + m->store.pt_offset(0, layer);
    c.state = m->store.state_dev();
    c.held_index = m->store.held_index(0, layer);
    c.seq_index = m->store.seq_index(0);
    c.capacity = static_cast<int>(std::min<long long>(m->store.capacity(), 0x7FFFFFFF));
    c.max_seq = m->max_seq;
    c.pos_dev = pos0_dev;
    c.n = n;
    QR_HIP(launch_page_claim(c, st));
    AppendArgs a{};
    a.pool = m->store.pool();
    a.page_table = m->store.page_table_dev() + m->store.pt_offset(0, layer);
    a.geom = m->store.geom();
    a.dtype = m->dtype;
    a.src[0] = rows_dev;
    a.row_len[0] = m->latent;
    a.src_stride = m->latent;
    a.src_dtype = src_dtype;
    a.pos0 = 0;
    a.n = n;
    a.pos_dev = pos0_dev;
    a.held_dev = m->store.state_dev() + c.held_index;
    a.max_seq = m->max_seq;
    QR_HIP(launch_append(a, st));
    m->store.mark_device_ahead();
    if (cap) m->store.mark_replayable();
    return QR_OK;
}

int qr_mla_attention_step_dev(qr_mla* m, int layer, const int* pos_dev, int heads, const float* q_tilde_dev,
                              const float* q_rope_dev, float scale, float* u_dev, void* stream) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_CHECK_ARG(pos_dev && q_tilde_dev && u_dev && (q_rope_dev || m->rope == 0), "null pos/q_tilde/q_rope/u pointer");
    QR_CHECK_ARG(m->split_set, "the latent's kv_lora/rope split is not set (qr_mla_set_rope)");
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(heads >= 1 && heads <= kMlaMaxHeads, "heads %d outside [1, %d]", heads, kMlaMaxHeads);
    QR_CHECK_ARG(m->store.capacity() >= 1, "the page pool is empty: nothing was appended or reserved");
    DeviceGuard dg(m->device);
    note_capture(m, static_cast<hipStream_t>(stream));
    return attention_dev(m, layer, 0, pos_dev, heads, q_tilde_dev, q_rope_dev, scale, u_dev,
                         static_cast<hipStream_t>(stream));
}

int qr_mla_attend_absorbed_step_dev(qr_mla* m, int layer, const int* pos_dev, int heads, int nope, int vdim,
                                    const float* q_dev, const void* kvb_dev, int kvb_format, float* out_dev,
                                    void* stream) {
    clear_error();
    QR_TRY(check_handle(m));
    QR_CHECK_ARG(pos_dev && q_dev && out_dev, "null pos / q / out pointer");
    QR_CHECK_ARG(m->split_set, "the latent's kv_lora/rope split is not set (qr_mla_set_rope)");
    QR_TRY(check_layer(m, layer));
    QR_CHECK_ARG(heads >= 1 && heads <= kMlaMaxHeads, "heads %d outside [1, %d]", heads, kMlaMaxHeads);
    QR_CHECK_ARG(m->store.capacity() >= 1, "the page pool is empty: nothing was appended or reserved");
    DeviceGuard dg(m->device);
    note_capture(m, static_cast<hipStream_t>(stream));
    return attend_absorbed_dev(m, layer, 0, pos_dev, heads, nope, vdim, q_dev, kvb_dev, kvb_format, out_dev,
                               static_cast<hipStream_t>(stream));
}

}  // extern "C"
