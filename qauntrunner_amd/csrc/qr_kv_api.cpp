// qr_kv.cpp -- C ABI of the paged GQA KV cache (PagedKvCache, PagedKvCache.cs:12-136).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "qr_chunk.hpp"
#include "qr_store.hpp"

namespace qr {
const char* last_error();
}

using namespace qr;

struct qr_kv {
    int device = 0;
    int layers = 0, heads = 0, kv_heads = 0, head_dim = 0, max_seq = 0, dtype = 0, max_batch = 0;
    int kv_dim = 0;
    PagedStore store;
    std::vector<int> seq_len;
    hipStream_t stream = nullptr;
    DevBuf stage;      // host <-> device staging of rows, queries and outputs
    DevBuf workspace;  // split-K partials
    DevBuf steppos;    // device positions of the queries of a device-position chunk (kMaxDecodeBatch ints)
    DevBuf counters;   // arrival counters of the in-kernel split merge (kDecodeCounters, zero between calls)
    hipEvent_t split_event = nullptr;  // benchmark instrumentation (qr_kv_set_split_event)
    void* scratch = nullptr;           // this device's decode scratch array (no-allocation calls)
    bool device_steps = false;         // the device copy of the page accounting is in use
};

namespace {

int check_handle(const qr_kv* kv) {
    if (!kv) {
        set_error("null qr_kv handle");
        return QR_ERR_INVALID_ARGUMENT;
    }
    return QR_OK;
}

int check_seq_layer(const qr_kv* kv, int seq_id, int layer) {
    QR_CHECK_ARG(seq_id >= 0 && seq_id < kv->max_batch, "seq_id %d outside [0, %d)", seq_id, kv->max_batch);
    QR_CHECK_ARG(layer >= 0 && layer < kv->layers, "layer %d outside [0, %d)", layer, kv->layers);
    return QR_OK;
}

int check_pos(const qr_kv* kv, int pos) {
    if (pos < 0 || pos >= kv->max_seq) {
        set_error("position %d outside [0, max_seq=%d)", pos, kv->max_seq);
        return QR_ERR_OUT_OF_RANGE;
    }
    return QR_OK;
}

int check_resident(const qr_kv* kv, int seq_id, int layer, int pos) {
    if (!kv->store.resident(seq_id, layer, pos)) {
        set_error("position %d of sequence %d layer %d was never appended (%d pages resident)", pos,
                  seq_id, layer, kv->store.pages_held(seq_id, layer));
        return QR_ERR_NOT_RESIDENT;
    }
    return QR_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Host view of the page accounting and SeqLen, read back from the device after
// device-side appends (a no-op otherwise).  A device-pointer call enqueued under stream
// capture skips the read-back (it would wait for the device): its checks then use the
// host accounting, which never runs ahead of the device's (pages and SeqLen only grow
// on the device), so they can reject a position the device already holds but never
// accept one it does not.
int sync_host(const qr_kv* ckv, hipStream_t stream = nullptr, bool device_call = false) {
    qr_kv* kv = const_cast<qr_kv*>(ckv);
    if (!kv->store.device_ahead()) return QR_OK;
    if (device_call && capturing(stream)) return QR_OK;
    DeviceGuard dg(kv->device);
    return kv->store.pull(kv->seq_len);
}

// A call enqueued under stream capture leaves the addresses of the pool, the split
// workspace and the position buffer in the graph: from then on the pool never moves
// (growing it is an error) and a workspace that grows keeps its old allocation alive
// for the graph's replays until the handle is destroyed.
void note_capture(qr_kv* kv, hipStream_t stream) {
    if (!capturing(stream)) return;
    kv->store.freeze();
    kv->workspace.keep_retired();
    kv->steppos.keep_retired();
}

// Device copy of the accounting after host-side changes (once device-side appends are in use).
int sync_device(qr_kv* kv, hipStream_t stream) {
    if (!kv->device_steps) return QR_OK;
    return kv->store.push(kv->seq_len, stream);
}

// Appends rows already on the device (src_dtype, row stride kv_dim).
int append_dev(qr_kv* kv, int seq_id, int layer, int pos0, int n, const void* k, const void* v,
               int k_len, int v_len, int src_dtype, hipStream_t stream) {
    QR_TRY(kv->store.ensure(seq_id, layer, pos0 + n, stream));
    AppendArgs a{};
    a.pool = kv->store.pool();
    a.page_table = kv->store.page_table_dev() + kv->store.pt_offset(seq_id, layer);
    a.geom = kv->store.geom();
    a.dtype = kv->dtype;
    a.src[0] = k;
    a.src[1] = v;
    a.row_len[0] = k_len;
    a.row_len[1] = v_len;
    a.src_stride = kv->kv_dim;
    a.src_dtype = src_dtype;
    a.pos0 = pos0;
    a.n = n;
    QR_HIP(launch_append(a, stream));
    int& sl = kv->seq_len[seq_id];
    sl = std::max(sl, pos0 + n);  // PagedKvCache.cs:68
    return sync_device(kv, stream);
}

// RoPE + append of n positions from device rows (fp32 k/v, q rotated in place).
int rope_append_dev(qr_kv* kv, int seq_id, int layer, int pos0, int n, float* q, const float* k,
                    const float* v, float theta, hipStream_t stream) {
    QR_TRY(kv->store.ensure(seq_id, layer, pos0 + n, stream));
    RopeAppendArgs a{};
    a.app.pool = kv->store.pool();
    a.app.page_table = kv->store.page_table_dev() + kv->store.pt_offset(seq_id, layer);
    a.app.geom = kv->store.geom();
    a.app.dtype = kv->dtype;
    a.app.src[0] = k;
    a.app.src[1] = v;
    a.app.row_len[0] = kv->kv_dim;
    a.app.row_len[1] = kv->kv_dim;
    a.app.src_stride = kv->kv_dim;
    a.app.src_dtype = QR_DTYPE_F32;
    a.app.pos0 = pos0;
    a.app.n = n;
    a.q = q;
    a.q_width = kv->heads * kv->head_dim;
    // freq_i = theta^(-2i/D) with the host libm powf, in the reference's fp32 order
    // (TransformerOps.cs:60: MathF.Pow(theta, -2f * i / headDim))
    const int half = kv->head_dim / 2;
    for (int i = 0; i < half; ++i) a.freq[i] = std::pow(theta, (-2.0f * static_cast<float>(i)) / static_cast<float>(kv->head_dim));
    QR_HIP(launch_rope_append(a, stream));
    int& sl = kv->seq_len[seq_id];
    sl = std::max(sl, pos0 + n);  // PagedKvCache.cs:68
    return sync_device(kv, stream);
}

// The split workspace may only grow outside stream capture.
int grow_workspace(qr_kv* kv, size_t bytes, hipStream_t st) {
    const size_t ws = std::max<size_t>(bytes, 256);
    if (ws > kv->workspace.size()) {
        QR_CHECK_ARG(!capturing(st), "the split workspace must grow to %zu bytes: make one call outside capture first", ws);
        QR_TRY(kv->workspace.ensure(ws));
    }
    return QR_OK;
}

// Runs decode entries (seq_ids[i], seq_len[i]) with device q/out rows.
int decode_dev(qr_kv* kv, int n, const int* seq_ids, const int* seq_len, int layer, const float* q,
               float* out, float scale, hipStream_t stream) {
    const size_t row = static_cast<size_t>(kv->heads) * kv->head_dim;
    for (int i0 = 0; i0 < n; i0 += kMaxDecodeBatch) {
        const int nb = std::min(kMaxDecodeBatch, n - i0);
        DecodeArgs a{};
        a.pool = kv->store.pool();
        a.page_table = kv->store.page_table_dev();
        a.geom = kv->store.geom();
        a.dtype = kv->dtype;
        a.heads = kv->heads;
        a.q = q + i0 * row;
        a.out = out + i0 * row;
        a.scale = scale;
        a.nb = nb;
        for (int i = 0; i < nb; ++i) {
            a.seq_len[i] = seq_len[i0 + i];
            a.pt_off[i] = kv->store.pt_offset(seq_ids[i0 + i], layer);
        }
        a.counters = static_cast<unsigned*>(kv->counters.get());
        const DecodePlan plan = plan_decode(a);
        QR_TRY(grow_workspace(kv, plan.workspace_bytes, stream));
        QR_HIP(launch_decode(a, plan, kv->workspace.get(), stream, kv->split_event));
    }
    return QR_OK;
}

int validate_batch(const qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos,
                   std::vector<int>& seq_len) {
    QR_CHECK_ARG(n >= 1, "batch size must be >= 1 (got %d)", n);
    QR_CHECK_ARG(seq_ids && pos, "null seq_ids/pos array");
    seq_len.resize(n);
    for (int i = 0; i < n; ++i) {
        QR_TRY(check_seq_layer(kv, seq_ids[i], layer));
        QR_TRY(check_pos(kv, pos[i]));
        QR_TRY(check_resident(kv, seq_ids[i], layer, pos[i]));
        seq_len[i] = pos[i] + 1;
    }
    return QR_OK;
}

}  // namespace

extern "C" {

int qr_abi_version(void) { return QR_ATTN_ABI_VERSION; }

const char* qr_last_error(void) { return qr::last_error(); }

const char* qr_status_name(int status) {
    switch (status) {
        case QR_OK: return "QR_OK";
        case QR_ERR_INVALID_ARGUMENT: return "QR_ERR_INVALID_ARGUMENT";
        case QR_ERR_OUT_OF_RANGE: return "QR_ERR_OUT_OF_RANGE";
        case QR_ERR_OUT_OF_MEMORY: return "QR_ERR_OUT_OF_MEMORY";
        case QR_ERR_HIP: return "QR_ERR_HIP";
        case QR_ERR_NOT_RESIDENT: return "QR_ERR_NOT_RESIDENT";
        default: return "QR_ERR_UNKNOWN";
    }
}

int qr_kv_create(qr_kv** out, int layers, int heads, int kv_heads, int head_dim, int max_seq,
                 int kv_dtype, int max_batch) {
    clear_error();
    QR_CHECK_ARG(out != nullptr, "null output handle pointer");
    *out = nullptr;
    QR_CHECK_ARG(layers >= 1, "layers must be >= 1 (got %d)", layers);
    QR_CHECK_ARG(heads >= 1 && kv_heads >= 1 && kv_heads <= heads,
                 "need 1 <= kv_heads <= heads (got heads=%d kv_heads=%d)", heads, kv_heads);
    QR_CHECK_ARG(head_dim >= 1 && head_dim <= kGenericMaxDim, "head_dim %d unsupported (1 to %d)", head_dim,
                 kGenericMaxDim);
    QR_CHECK_ARG(max_seq >= 1, "max_seq must be >= 1 (got %d)", max_seq);
    QR_CHECK_ARG(dtype_valid(kv_dtype), "unknown kv dtype %d", kv_dtype);
    QR_CHECK_ARG(max_batch >= 1, "max_batch must be >= 1 (got %d)", max_batch);
    const long long pt_entries = static_cast<long long>(max_batch) * layers * ((max_seq + kPageTokens - 1) / kPageTokens);
    QR_CHECK_ARG(pt_entries < (1LL << 31), "page table of %lld entries is too large", pt_entries);

    qr_kv* kv = new (std::nothrow) qr_kv();
    if (!kv) {
        set_error("host allocation of the handle failed");
        return QR_ERR_OUT_OF_MEMORY;
    }
    kv->layers = layers;
    kv->heads = heads;
    kv->kv_heads = kv_heads;
    kv->head_dim = head_dim;
    kv->max_seq = max_seq;
    kv->dtype = kv_dtype;
    kv->max_batch = max_batch;
    kv->kv_dim = kv_heads * head_dim;
    kv->seq_len.assign(max_batch, 0);
    int st = QR_OK;
    if (hipGetDevice(&kv->device) != hipSuccess) {
        set_error("no HIP device available");
        st = QR_ERR_HIP;
    }
    if (st == QR_OK) {
        PageGeom g{2, kv_heads, head_dim};
        g.mfma_layout = kv_mfma_layout(kv_dtype, head_dim) ? 1 : 0;
        st = kv->store.init(g, kv_dtype, layers, max_batch, max_seq);
    }
    if (st == QR_OK) st = decode_scratch_address(kv->device, &kv->scratch);
    if (st == QR_OK) st = kv->steppos.ensure(kMaxDecodeBatch * sizeof(int));
    if (st == QR_OK) st = kv->counters.ensure(kDecodeCounterBytes, true);
    if (st == QR_OK && hipStreamCreateWithFlags(&kv->stream, hipStreamNonBlocking) != hipSuccess) {
        set_error("hipStreamCreateWithFlags failed");
        st = QR_ERR_HIP;
    }
    if (st != QR_OK) {
        if (kv->stream) (void)hipStreamDestroy(kv->stream);
        delete kv;
        return st;
    }
    *out = kv;
    return QR_OK;
}

int qr_kv_destroy(qr_kv* kv) {
    clear_error();
    if (!kv) return QR_OK;
    DeviceGuard dg(kv->device);
    (void)hipStreamSynchronize(kv->stream);
    (void)hipStreamDestroy(kv->stream);
    delete kv;
    return QR_OK;
}

int qr_kv_reserve(qr_kv* kv, int pages) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    DeviceGuard dg(kv->device);
    return kv->store.reserve(pages);
}

int qr_kv_append(qr_kv* kv, int seq_id, int layer, int pos, const float* k, int k_len, const float* v,
                 int v_len) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_TRY(check_pos(kv, pos));
    QR_CHECK_ARG(k_len >= 0 && v_len >= 0, "negative row length");
    QR_CHECK_ARG((k || k_len == 0) && (v || v_len == 0), "null k/v row");
    if (k_len > kv->kv_dim || v_len > kv->kv_dim) {
        set_error("row of %d/%d floats is longer than kv_dim=%d", k_len, v_len, kv->kv_dim);
        return QR_ERR_OUT_OF_RANGE;
    }
    DeviceGuard dg(kv->device);
    const size_t bytes = static_cast<size_t>(kv->kv_dim) * 4;
    QR_TRY(kv->stage.ensure(2 * bytes));
    char* st = static_cast<char*>(kv->stage.get());
    if (k_len) QR_HIP(hipMemcpyAsync(st, k, k_len * 4, hipMemcpyHostToDevice, kv->stream));
    if (v_len) QR_HIP(hipMemcpyAsync(st + bytes, v, v_len * 4, hipMemcpyHostToDevice, kv->stream));
    QR_TRY(append_dev(kv, seq_id, layer, pos, 1, st, st + bytes, k_len, v_len, QR_DTYPE_F32, kv->stream));
    QR_HIP(hipStreamSynchronize(kv->stream));
    return QR_OK;
}

int qr_kv_append_range(qr_kv* kv, int seq_id, int layer, int pos0, int n, const void* k, const void* v,
                       int src_dtype) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(dtype_valid(src_dtype), "unknown source dtype %d", src_dtype);
    QR_CHECK_ARG(n >= 0, "negative row count %d", n);
    QR_CHECK_ARG(n == 0 || (k && v), "null k/v rows");
    if (n == 0) return QR_OK;
    QR_TRY(check_pos(kv, pos0));
    QR_TRY(check_pos(kv, pos0 + n - 1));
    DeviceGuard dg(kv->device);
    const size_t bytes = static_cast<size_t>(n) * kv->kv_dim * dtype_size(src_dtype);
    QR_TRY(kv->stage.ensure(2 * bytes));
    char* st = static_cast<char*>(kv->stage.get());
    QR_HIP(hipMemcpyAsync(st, k, bytes, hipMemcpyHostToDevice, kv->stream));
    QR_HIP(hipMemcpyAsync(st + bytes, v, bytes, hipMemcpyHostToDevice, kv->stream));
    QR_TRY(append_dev(kv, seq_id, layer, pos0, n, st, st + bytes, kv->kv_dim, kv->kv_dim, src_dtype, kv->stream));
    QR_HIP(hipStreamSynchronize(kv->stream));
    return QR_OK;
}

int qr_kv_append_range_dev(qr_kv* kv, int seq_id, int layer, int pos0, int n, const void* k_dev,
                           const void* v_dev, int src_dtype, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv, as_stream(stream), true));
    note_capture(kv, as_stream(stream));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(dtype_valid(src_dtype), "unknown source dtype %d", src_dtype);
    QR_CHECK_ARG(n >= 0, "negative row count %d", n);
    QR_CHECK_ARG(n == 0 || (k_dev && v_dev), "null k/v rows");
    if (n == 0) return QR_OK;
    QR_TRY(check_pos(kv, pos0));
    QR_TRY(check_pos(kv, pos0 + n - 1));
    DeviceGuard dg(kv->device);
    return append_dev(kv, seq_id, layer, pos0, n, k_dev, v_dev, kv->kv_dim, kv->kv_dim, src_dtype,
                      as_stream(stream));
}

int qr_kv_append_rope(qr_kv* kv, int seq_id, int layer, int pos, float* q, const float* k, const float* v,
                      float theta) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_TRY(check_pos(kv, pos));
    QR_CHECK_ARG(q && k && v, "null q/k/v row");
    DeviceGuard dg(kv->device);
    const size_t kbytes = static_cast<size_t>(kv->kv_dim) * 4;
    const size_t qbytes = static_cast<size_t>(kv->heads) * kv->head_dim * 4;
    QR_TRY(kv->stage.ensure(2 * kbytes + qbytes + 512));
    char* st = static_cast<char*>(kv->stage.get());
    float* dk = reinterpret_cast<float*>(st);
    float* dv = reinterpret_cast<float*>(st + kbytes);
    float* dq = reinterpret_cast<float*>(st + 2 * kbytes);
    QR_HIP(hipMemcpyAsync(dk, k, kbytes, hipMemcpyHostToDevice, kv->stream));
    QR_HIP(hipMemcpyAsync(dv, v, kbytes, hipMemcpyHostToDevice, kv->stream));
    QR_HIP(hipMemcpyAsync(dq, q, qbytes, hipMemcpyHostToDevice, kv->stream));
    QR_TRY(rope_append_dev(kv, seq_id, layer, pos, 1, dq, dk, dv, theta, kv->stream));
    QR_HIP(hipMemcpyAsync(q, dq, qbytes, hipMemcpyDeviceToHost, kv->stream));
    QR_HIP(hipStreamSynchronize(kv->stream));
    return QR_OK;
}

int qr_kv_append_rope_dev(qr_kv* kv, int seq_id, int layer, int pos0, int n, float* q_dev, const float* k_dev,
                          const float* v_dev, float theta, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv, as_stream(stream), true));
    note_capture(kv, as_stream(stream));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(n >= 0, "negative row count %d", n);
    QR_CHECK_ARG(n == 0 || (k_dev && v_dev), "null k/v rows");
    if (n == 0) return QR_OK;
    QR_TRY(check_pos(kv, pos0));
    QR_TRY(check_pos(kv, pos0 + n - 1));
    QR_CHECK_ARG(((reinterpret_cast<uintptr_t>(q_dev) | reinterpret_cast<uintptr_t>(k_dev) |
                   reinterpret_cast<uintptr_t>(v_dev)) & 15) == 0, "q/k/v rows must be 16-byte aligned");
    DeviceGuard dg(kv->device);
    return rope_append_dev(kv, seq_id, layer, pos0, n, q_dev, k_dev, v_dev, theta, as_stream(stream));
}

int qr_kv_attention(qr_kv* kv, int seq_id, int layer, int pos, const float* q, float* attn, float scale) {
    return qr_kv_attention_batch(kv, 1, &seq_id, layer, &pos, q, attn, scale);
}

int qr_kv_attention_batch(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos, const float* q,
                          float* attn, float scale) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_CHECK_ARG(q && attn, "null q/attn pointer");
    std::vector<int> seq_len;
    QR_TRY(validate_batch(kv, n, seq_ids, layer, pos, seq_len));
    DeviceGuard dg(kv->device);
    const size_t bytes = static_cast<size_t>(n) * kv->heads * kv->head_dim * 4;
    QR_TRY(kv->stage.ensure(2 * bytes));
    float* dq = static_cast<float*>(kv->stage.get());
    float* dout = reinterpret_cast<float*>(static_cast<char*>(kv->stage.get()) + bytes);
    QR_HIP(hipMemcpyAsync(dq, q, bytes, hipMemcpyHostToDevice, kv->stream));
    QR_TRY(decode_dev(kv, n, seq_ids, seq_len.data(), layer, dq, dout, scale, kv->stream));
    QR_HIP(hipMemcpyAsync(attn, dout, bytes, hipMemcpyDeviceToHost, kv->stream));
    QR_HIP(hipStreamSynchronize(kv->stream));
    return QR_OK;
}

int qr_kv_attention_dev(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos, const float* q_dev,
                        float* attn_dev, float scale, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv, as_stream(stream), true));
    note_capture(kv, as_stream(stream));
    QR_CHECK_ARG(q_dev && attn_dev, "null q/attn pointer");
    std::vector<int> seq_len;
    QR_TRY(validate_batch(kv, n, seq_ids, layer, pos, seq_len));
    DeviceGuard dg(kv->device);
    return decode_dev(kv, n, seq_ids, seq_len.data(), layer, q_dev, attn_dev, scale, as_stream(stream));
}

int qr_kv_attention_dev_noalloc(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos,
                                const float* q_dev, float* attn_dev, float scale, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv, as_stream(stream), true));
    note_capture(kv, as_stream(stream));
    QR_CHECK_ARG(q_dev && attn_dev, "null q/attn pointer");
    QR_CHECK_ARG(n >= 1 && n <= kMaxDecodeBatch, "batch size %d outside [1, %d] for the no-allocation call", n,
                 kMaxDecodeBatch);
    QR_CHECK_ARG(seq_ids && pos, "null seq_ids/pos array");
    DecodeArgs a{};  // fixed-size descriptor: no host or device allocation on this path
    for (int i = 0; i < n; ++i) {
        QR_TRY(check_seq_layer(kv, seq_ids[i], layer));
        QR_TRY(check_pos(kv, pos[i]));
        QR_TRY(check_resident(kv, seq_ids[i], layer, pos[i]));
        a.seq_len[i] = pos[i] + 1;
        a.pt_off[i] = kv->store.pt_offset(seq_ids[i], layer);
    }
    DeviceGuard dg(kv->device);
    a.pool = kv->store.pool();
    a.page_table = kv->store.page_table_dev();
    a.geom = kv->store.geom();
    a.dtype = kv->dtype;
    a.heads = kv->heads;
    a.q = q_dev;
    a.out = attn_dev;
    a.scale = scale;
    a.nb = n;
    // the scratch array holds the arrival counters, then the split partials
    a.counters = static_cast<unsigned*>(kv->scratch);
    const DecodePlan plan = plan_decode(a);
    if (plan.workspace_bytes > kDecodeScratchBytes - kDecodeCounterBytes) {
        set_error("split partials of %zu bytes exceed the %zu bytes the no-allocation call's scratch holds "
                  "(fewer entries or shorter sequences per call, or qr_kv_attention_dev)",
                  plan.workspace_bytes, kDecodeScratchBytes - kDecodeCounterBytes);
        return QR_ERR_OUT_OF_RANGE;
    }
    QR_HIP(launch_decode(a, plan, static_cast<char*>(kv->scratch) + kDecodeCounterBytes, as_stream(stream),
                         kv->split_event));
    return QR_OK;
}

namespace {
int chunk_common(qr_kv* kv, int seq_id, int layer, int pos0, int nq, const void* q, int q_dtype,
                 float* attn, bool q_is_dev, bool out_is_dev, float scale, hipStream_t stream) {
    QR_TRY(check_handle(kv));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(q && attn, "null q/attn pointer");
    QR_CHECK_ARG(dtype_valid(q_dtype), "unknown q dtype %d", q_dtype);
    QR_CHECK_ARG(nq >= 1, "nq must be >= 1 (got %d)", nq);
    QR_TRY(check_pos(kv, pos0));
    QR_TRY(check_pos(kv, pos0 + nq - 1));
    QR_TRY(check_resident(kv, seq_id, layer, pos0 + nq - 1));
    DeviceGuard dg(kv->device);
    const size_t rowf = static_cast<size_t>(kv->heads) * kv->head_dim;
    const size_t qbytes = nq * rowf * dtype_size(q_dtype);
    const size_t fbytes = nq * rowf * 4;
    // staging: [raw q (host path)] [fp32 q] [fp32 out (host path)]
    QR_TRY(kv->stage.ensure(qbytes + 2 * fbytes + 512));
    char* st = static_cast<char*>(kv->stage.get());
    const void* qsrc = q;
    if (!q_is_dev) {
        QR_HIP(hipMemcpyAsync(st, q, qbytes, hipMemcpyHostToDevice, stream));
        qsrc = st;
    }
    float* q32 = reinterpret_cast<float*>(st + ((qbytes + 255) & ~size_t(255)));
    float* dout = out_is_dev ? attn : q32 + nq * rowf;
    if (chunk_mfma_eligible(kv->dtype, kv->head_dim, kv->heads, kv->kv_heads)) {
        // MFMA tiles read each K/V tile once for a block of queries
        ChunkArgs c{};
        c.pool = kv->store.pool();
        c.page_table = kv->store.page_table_dev() + kv->store.pt_offset(seq_id, layer);
        c.geom = kv->store.geom();
        c.kv_dtype = kv->dtype;
        c.heads = kv->heads;
        c.pos0 = pos0;
        c.nq = nq;
        c.q = qsrc;
        c.q_dtype = q_dtype;
        c.out = dout;
        c.scale = scale;
        const ChunkPlan plan = plan_chunk(c);
        QR_TRY(grow_workspace(kv, plan.workspace_bytes, stream));
        QR_HIP(launch_chunk(c, plan, kv->workspace.get(), stream, kv->split_event));
    } else {
        // exact fp32 path: every query is one decode entry with its causal length; the
        // decode kernels read fp32 queries, so 16-bit ones are widened first (the MFMA
        // branch above reads them in their own type)
        const float* qf = static_cast<const float*>(qsrc);
        if (q_dtype != QR_DTYPE_F32) {
            QR_HIP(launch_widen(qsrc, q_dtype, q32, static_cast<long long>(nq) * rowf, stream));
            qf = q32;
        }
        std::vector<int> ids(nq, seq_id), lens(nq);
        for (int i = 0; i < nq; ++i) lens[i] = pos0 + i + 1;
        QR_TRY(decode_dev(kv, nq, ids.data(), lens.data(), layer, qf, dout, scale, stream));
    }
    if (!out_is_dev) {
        QR_HIP(hipMemcpyAsync(attn, dout, fbytes, hipMemcpyDeviceToHost, stream));
        QR_HIP(hipStreamSynchronize(stream));
    }
    return QR_OK;
}
}  // namespace

int qr_kv_attention_chunk(qr_kv* kv, int seq_id, int layer, int pos0, int nq, const void* q, int q_dtype,
                          float* attn, float scale) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    return chunk_common(kv, seq_id, layer, pos0, nq, q, q_dtype, attn, false, false, scale, kv->stream);
}

int qr_kv_attention_chunk_dev(qr_kv* kv, int seq_id, int layer, int pos0, int nq, const void* q_dev,
                              int q_dtype, float* attn_dev, float scale, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv, as_stream(stream), true));
    note_capture(kv, as_stream(stream));
    return chunk_common(kv, seq_id, layer, pos0, nq, q_dev, q_dtype, attn_dev, true, true, scale,
                        as_stream(stream));
}

int qr_kv_decode_plan(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos, int* split_tokens,
                      int* splits) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_CHECK_ARG(split_tokens && splits, "null output pointer");
    std::vector<int> seq_len;
    QR_TRY(validate_batch(kv, n, seq_ids, layer, pos, seq_len));
    DeviceGuard dg(kv->device);
    DecodeArgs a{};
    a.geom = kv->store.geom();
    a.dtype = kv->dtype;
    a.heads = kv->heads;
    a.nb = std::min(n, kMaxDecodeBatch);
    for (int i = 0; i < a.nb; ++i) a.seq_len[i] = seq_len[i];
    const DecodePlan plan = plan_decode(a);
    *split_tokens = plan.split_tokens;
    *splits = plan.max_splits;
    return QR_OK;
}

int qr_kv_set_split_event(qr_kv* kv, void* event) {
    clear_error();
    QR_TRY(check_handle(kv));
    kv->split_event = static_cast<hipEvent_t>(event);
    return QR_OK;
}

int qr_kv_reset(qr_kv* kv, int seq_id) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    if (seq_id < 0) {
        std::fill(kv->seq_len.begin(), kv->seq_len.end(), 0);
    } else {
        QR_CHECK_ARG(seq_id < kv->max_batch, "seq_id %d outside [0, %d)", seq_id, kv->max_batch);
        kv->seq_len[seq_id] = 0;
    }
    if (kv->device_steps) {
        DeviceGuard dg(kv->device);
        QR_TRY(sync_device(kv, kv->stream));
        QR_HIP(hipStreamSynchronize(kv->stream));
    }
    return QR_OK;
}

int qr_kv_truncate(qr_kv* kv, int seq_id, int len) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_CHECK_ARG(seq_id >= 0 && seq_id < kv->max_batch, "seq_id %d outside [0, %d)", seq_id, kv->max_batch);
    if (len < kv->seq_len[seq_id]) kv->seq_len[seq_id] = len;  // PagedKvCache.cs:76
    if (kv->device_steps) {
        DeviceGuard dg(kv->device);
        QR_TRY(sync_device(kv, kv->stream));
        QR_HIP(hipStreamSynchronize(kv->stream));
    }
    return QR_OK;
}

int qr_kv_seq_len(const qr_kv* kv, int seq_id, int* out) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_CHECK_ARG(out, "null output pointer");
    QR_CHECK_ARG(seq_id >= 0 && seq_id < kv->max_batch, "seq_id %d outside [0, %d)", seq_id, kv->max_batch);
    *out = kv->seq_len[seq_id];
    return QR_OK;
}

int qr_kv_bytes_used(const qr_kv* kv, long long* out) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_CHECK_ARG(out, "null output pointer");
    *out = kv->store.bytes_used();
    return QR_OK;
}

int qr_kv_bytes_per_token(const qr_kv* kv, long long* out) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_CHECK_ARG(out, "null output pointer");
    *out = static_cast<long long>(kv->kv_dim) * dtype_size(kv->dtype) * 2 * kv->layers;
    return QR_OK;
}

int qr_kv_read(qr_kv* kv, int seq_id, int layer, int pos0, int n, void* k_out, void* v_out) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(sync_host(kv));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(n >= 0, "negative row count %d", n);
    QR_CHECK_ARG(n == 0 || (k_out && v_out), "null output rows");
    if (n == 0) return QR_OK;
    QR_TRY(check_pos(kv, pos0));
    QR_TRY(check_pos(kv, pos0 + n - 1));
    QR_TRY(check_resident(kv, seq_id, layer, pos0 + n - 1));
    DeviceGuard dg(kv->device);
    const size_t bytes = static_cast<size_t>(n) * kv->kv_dim * dtype_size(kv->dtype);
    QR_TRY(kv->stage.ensure(2 * bytes));
    char* st = static_cast<char*>(kv->stage.get());
    GatherArgs g{};
    g.pool = kv->store.pool();
    g.page_table = kv->store.page_table_dev() + kv->store.pt_offset(seq_id, layer);
    g.geom = kv->store.geom();
    g.dtype = kv->dtype;
    g.dst[0] = st;
    g.dst[1] = st + bytes;
    g.pos0 = pos0;
    g.n = n;
    g.to_f32 = 0;
    QR_HIP(launch_gather(g, kv->stream));
    QR_HIP(hipMemcpyAsync(k_out, st, bytes, hipMemcpyDeviceToHost, kv->stream));
    QR_HIP(hipMemcpyAsync(v_out, st + bytes, bytes, hipMemcpyDeviceToHost, kv->stream));
    QR_HIP(hipStreamSynchronize(kv->stream));
    return QR_OK;
}

}  // extern "C"

namespace {

// Ensure + RoPE + Append of n rows at the device positions *pos_dev .. *pos_dev + n - 1
// (the single-position and the chunk step calls).
int rope_step_dev(qr_kv* kv, int seq_id, int layer, int n, const int* pos_dev, float* q_dev, const float* k_dev,
                  const float* v_dev, float theta, hipStream_t st) {
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(pos_dev && k_dev && v_dev, "null pos/k/v pointer");
    // checked before the page claim is enqueued: a rejected append must leave the
    // device accounting as it was
    QR_CHECK_ARG(rope_generic(kv->head_dim) ||
                     rope_items_per_thread(kv->kv_heads + (q_dev ? kv->heads : 0), kv->head_dim) <= kRopeMaxItems,
                 "device-position RoPE appends take at most %d dims of K and q per position (got %d)",
                 kRopeThreads * kRopeMaxItems * 8, (kv->kv_heads + (q_dev ? kv->heads : 0)) * kv->head_dim);
    DeviceGuard dg(kv->device);
    const bool cap = capturing(st);
    note_capture(kv, st);
    if (!kv->device_steps) {
        // first device-side append: the device copy starts from the host accounting
        QR_CHECK_ARG(!cap, "the first device-side append of a cache must run outside stream capture");
        QR_TRY(sync_host(kv));
        kv->device_steps = true;
        QR_TRY(kv->store.push(kv->seq_len, st));
    }
    if (kv->store.capacity() < 1) {
        QR_CHECK_ARG(!cap, "the page pool is empty: reserve pages before capturing device-side appends");
        QR_TRY(kv->store.reserve(16));
    }
    PageClaimArgs c{};
    c.page_table = const_cast<int*>(kv->store.page_table_dev()) + kv->store.pt_offset(seq_id, layer);
    c.state = kv->store.state_dev();
    c.held_index = kv->store.held_index(seq_id, layer);
    c.seq_index = kv->store.seq_index(seq_id);
    c.capacity = static_cast<int>(std::min<long long>(kv->store.capacity(), 0x7FFFFFFF));
    c.max_seq = kv->max_seq;
    c.pos_dev = pos_dev;
    c.n = n;
    QR_HIP(launch_page_claim(c, st));
    RopeAppendArgs a{};
    a.app.pool = kv->store.pool();
    a.app.page_table = kv->store.page_table_dev() + kv->store.pt_offset(seq_id, layer);
    a.app.geom = kv->store.geom();
    a.app.dtype = kv->dtype;
    a.app.src[0] = k_dev;
    a.app.src[1] = v_dev;
    a.app.row_len[0] = kv->kv_dim;
    a.app.row_len[1] = kv->kv_dim;
    a.app.src_stride = kv->kv_dim;
    a.app.src_dtype = QR_DTYPE_F32;
    a.app.pos0 = 0;
    a.app.n = n;
    a.app.pos_dev = pos_dev;
    a.app.held_dev = kv->store.state_dev() + c.held_index;
    a.app.max_seq = kv->max_seq;
    a.q = q_dev;
    a.q_width = kv->heads * kv->head_dim;
    const int half = kv->head_dim / 2;
    for (int i = 0; i < half; ++i) a.freq[i] = std::pow(theta, (-2.0f * static_cast<float>(i)) / static_cast<float>(kv->head_dim));
    QR_HIP(launch_rope_append(a, st));
    kv->store.mark_device_ahead();
    if (cap) kv->store.mark_replayable();
    return QR_OK;
}

// Decode where entry i attends positions 0..pos_dev[i] (read on the device).
int attention_step(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos_dev, const float* q_dev,
                   float* attn_dev, float scale, hipStream_t st) {
    QR_CHECK_ARG(kv->store.capacity() >= 1, "the page pool is empty: nothing was appended or reserved");
    DecodeArgs a{};
    for (int i = 0; i < n; ++i) {
        QR_TRY(check_seq_layer(kv, seq_ids[i], layer));
        a.seq_len[i] = kv->max_seq;  // bound of the plan; the kernels read the positions
        a.pt_off[i] = kv->store.pt_offset(seq_ids[i], layer);
    }
    a.pool = kv->store.pool();
    a.page_table = kv->store.page_table_dev();
    a.geom = kv->store.geom();
    a.dtype = kv->dtype;
    a.heads = kv->heads;
    a.q = q_dev;
    a.out = attn_dev;
    a.scale = scale;
    a.nb = n;
    a.pos_dev = pos_dev;
    a.counters = static_cast<unsigned*>(kv->counters.get());
    const DecodePlan plan = plan_decode(a);
    QR_TRY(grow_workspace(kv, plan.workspace_bytes, st));
    QR_HIP(launch_decode(a, plan, kv->workspace.get(), st, nullptr));
    return QR_OK;
}

}  // namespace

extern "C" {

int qr_kv_append_rope_step_dev(qr_kv* kv, int seq_id, int layer, const int* pos_dev, float* q_dev,
                               const float* k_dev, const float* v_dev, float theta, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    return rope_step_dev(kv, seq_id, layer, 1, pos_dev, q_dev, k_dev, v_dev, theta, as_stream(stream));
}

int qr_kv_append_rope_chunk_step_dev(qr_kv* kv, int seq_id, int layer, int nq, const int* pos0_dev, float* q_dev,
                                     const float* k_dev, const float* v_dev, float theta, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_CHECK_ARG(nq >= 1 && nq <= kv->max_seq, "nq %d outside [1, %d]", nq, kv->max_seq);
    return rope_step_dev(kv, seq_id, layer, nq, pos0_dev, q_dev, k_dev, v_dev, theta, as_stream(stream));
}

int qr_kv_attention_step_dev(qr_kv* kv, int n, const int* seq_ids, int layer, const int* pos_dev,
                             const float* q_dev, float* attn_dev, float scale, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_CHECK_ARG(q_dev && attn_dev && pos_dev, "null q/attn/pos pointer");
    QR_CHECK_ARG(n >= 1 && n <= kMaxDecodeBatch, "batch size %d outside [1, %d] for device positions", n,
                 kMaxDecodeBatch);
    QR_CHECK_ARG(seq_ids, "null seq_ids array");
    DeviceGuard dg(kv->device);
    note_capture(kv, as_stream(stream));
    return attention_step(kv, n, seq_ids, layer, pos_dev, q_dev, attn_dev, scale, as_stream(stream));
}

int qr_kv_attention_chunk_step_dev(qr_kv* kv, int seq_id, int layer, int nq, const int* pos0_dev, const void* q_dev,
                                   int q_dtype, float* attn_dev, float scale, void* stream) {
    clear_error();
    QR_TRY(check_handle(kv));
    QR_TRY(check_seq_layer(kv, seq_id, layer));
    QR_CHECK_ARG(q_dev && attn_dev && pos0_dev, "null q/attn/pos pointer");
    QR_CHECK_ARG(dtype_valid(q_dtype), "unknown q dtype %d", q_dtype);
    QR_CHECK_ARG(nq >= 1 && nq <= kv->max_seq, "nq %d outside [1, %d]", nq, kv->max_seq);
    DeviceGuard dg(kv->device);
    const hipStream_t st = as_stream(stream);
    note_capture(kv, st);
    QR_CHECK_ARG(kv->store.capacity() >= 1, "the page pool is empty: nothing was appended or reserved");
    if (chunk_mfma_eligible(kv->dtype, kv->head_dim, kv->heads, kv->kv_heads)) {
        ChunkArgs c{};
        c.pool = kv->store.pool();
        c.page_table = kv->store.page_table_dev() + kv->store.pt_offset(seq_id, layer);
        c.geom = kv->store.geom();
        c.kv_dtype = kv->dtype;
        c.heads = kv->heads;
        c.pos0 = kv->max_seq - nq;  // bound of the plan; the kernels read the position
        c.pos0_dev = pos0_dev;
        c.nq = nq;
        c.q = q_dev;
        c.q_dtype = q_dtype;
        c.out = attn_dev;
        c.scale = scale;
        const ChunkPlan plan = plan_chunk(c);
        QR_TRY(grow_workspace(kv, plan.workspace_bytes, st));
        QR_HIP(launch_chunk(c, plan, kv->workspace.get(), st, nullptr));
        return QR_OK;
    }
    // other caches: one decode entry per query, its position written on the device
    QR_CHECK_ARG(q_dtype == QR_DTYPE_F32, "device-position chunks on this cache take fp32 queries (got dtype %d)", q_dtype);
    QR_CHECK_ARG(nq <= kMaxDecodeBatch, "device-position chunks on this cache take at most %d queries (got %d)",
                 kMaxDecodeBatch, nq);
    int* pos = static_cast<int*>(kv->steppos.get());
    QR_HIP(launch_positions(pos, pos0_dev, nq, st));
    const std::vector<int> ids(nq, seq_id);
    return attention_step(kv, nq, ids.data(), layer, pos, static_cast<const float*>(q_dev), attn_dev, scale, st);
}

}  // extern "C"

