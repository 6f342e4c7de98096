// qr_model.cpp -- .qw weight files served from HBM: ModelStore (Memory/ModelStore.cs) and the
// layer prefetch pipeline (Runtime/PrefetchPipeline.cs), MI355X side.
//
// The reference reads layer N+1 from disk into a pinned ping-pong buffer on a background task
// while layer N computes.  Here each of the two slots is an HBM buffer with its own copy stream:
// a worker thread reads the layer's tensors with positional reads into a pinned host buffer
// (hipHostMalloc) and queues one hipMemcpyAsync on the slot's stream.  Acquire makes the
// caller's stream wait for that upload on the GPU; the host waits only while the file read
// is still running.  GPU compute is asynchronous, so before a slot is overwritten its copy
// stream waits for the work that read the slot's previous layer: from the point where Release
// was called on each stream that acquired it, else from the point of the next Begin of that
// slot.  make_resident uploads every tensor once (one allocation); Acquire then never waits.
// On a 288 GB part that is the normal case.
#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "qr_common.hpp"
#include "qr_store.hpp"

using namespace qr;

namespace {

// ------------------------------------------------------------------ minimal JSON reader
// Enough of JSON for the .qw header: objects, arrays, strings, numbers, literals.
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    double num = 0;
    long long inum = 0;
    bool is_int = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const char* k) const {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    bool ok = true;
    int depth = 0;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if (static_cast<size_t>(end - p) < n || memcmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    bool string(std::string& out) {
        if (p >= end || *p != '"') return false;
        ++p;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) return false;
                switch (*p) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {  // \uXXXX: kept as UTF-8 for the BMP
                    if (end - p < 5) return false;
                    unsigned v = 0;
                    for (int i = 1; i <= 4; ++i) {
                        const char c = p[i];
                        v <<= 4;
                        if (c >= '0' && c <= '9') v |= c - '0';
                        else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
                        else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
                        else return false;
                    }
                    p += 4;
                    if (v < 0x80) out += static_cast<char>(v);
                    else if (v < 0x800) {
                        out += static_cast<char>(0xC0 | (v >> 6));
                        out += static_cast<char>(0x80 | (v & 0x3F));
                    } else {
                        out += static_cast<char>(0xE0 | (v >> 12));
                        out += static_cast<char>(0x80 | ((v >> 6) & 0x3F));
                        out += static_cast<char>(0x80 | (v & 0x3F));
                    }
                    break;
                }
                default: return false;
                }
                ++p;
            } else {
                out += *p++;
            }
        }
        if (p >= end) return false;
        ++p;
        return true;
    }
    bool value(Json& v) {
        if (++depth > 64) return false;
        ws();
        if (p >= end) return false;
        bool r = true;
        if (*p == '{') {
            v.kind = Json::Obj;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
            } else {
                for (;;) {
                    ws();
                    std::string k;
                    if (!string(k)) { r = false; break; }
                    ws();
                    if (p >= end || *p != ':') { r = false; break; }
                    ++p;
                    Json child;
                    if (!value(child)) { r = false; break; }
                    v.obj.emplace_back(std::move(k), std::move(child));
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == '}') { ++p; break; }
                    r = false;
                    break;
                }
            }
        } else if (*p == '[') {
            v.kind = Json::Arr;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
            } else {
                for (;;) {
                    Json child;
                    if (!value(child)) { r = false; break; }
                    v.arr.push_back(std::move(child));
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == ']') { ++p; break; }
                    r = false;
                    break;
                }
            }
        } else if (*p == '"') {
            v.kind = Json::Str;
            r = string(v.str);
        } else if (lit("true")) {
            v.kind = Json::Bool;
            v.num = 1;
        } else if (lit("false")) {
            v.kind = Json::Bool;
        } else if (lit("null")) {
            v.kind = Json::Null;
        } else {
            const char* s = p;
            while (p < end && (strchr("+-0123456789.eE", *p) != nullptr)) ++p;
            if (p == s) return false;
            const std::string t(s, p);
            v.kind = Json::Num;
            char* e = nullptr;
            v.num = strtod(t.c_str(), &e);
            if (e != t.c_str() + t.size()) return false;
            if (t.find_first_of(".eE") == std::string::npos) {
                v.is_int = true;
                v.inum = strtoll(t.c_str(), nullptr, 10);
            }
        }
        --depth;
        return r;
    }
};

bool as_int(const Json* j, long long* out) {
    if (!j || j->kind != Json::Num || !j->is_int) return false;
    *out = j->inum;
    return true;
}

// ------------------------------------------------------------------ model
struct Tensor {
    std::string name;
    std::vector<long long> dims;
    int format = 0;
    long long file_offset = 0;  // absolute
    long long bytes = 0;
};

constexpr size_t kAlign = 256;  // tensor alignment inside the HBM slots and the resident copy
// File read + upload unit of a staged layer, and reader threads per staged layer.  The
// environment variables QR_PREFETCH_READERS (1..64) and QR_PREFETCH_CHUNK_MB (1..256)
// override them when a handle is opened.
constexpr size_t kReadChunk = 2u << 20;
constexpr size_t kReadThreads = 16;

size_t env_size(const char* name, size_t dflt, size_t lo, size_t hi) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    char* end = nullptr;
    const unsigned long long x = strtoull(v, &end, 10);
    return (*end == '\0' && x >= lo && x <= hi) ? static_cast<size_t>(x) : dflt;
}

struct ReadChunk {
    size_t slot_offset;
    long long file_offset;
    size_t bytes;
};
size_t align_up(size_t b) { return (b + kAlign - 1) / kAlign * kAlign; }

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace

struct qr_model {
    std::string path;
    int fd = -1;
    std::vector<Tensor> tensors;           // header order (the reference's Tensors.Keys order)
    std::map<std::string, size_t> index;   // name -> position in `tensors`

    long long budget = 0;                  // PrefetchPipeline budget; 0 = disabled
    size_t read_chunk = kReadChunk;
    size_t read_threads = kReadThreads;
    int device = -1;
    bool device_ready = false;

    struct Slot {
        int for_layer = INT_MIN;
        bool staged = false;
        std::thread task;
        hipStream_t stream = nullptr;      // this slot's copy stream
        void* pinned = nullptr;
        size_t pinned_cap = 0;
        void* dev = nullptr;
        size_t dev_cap = 0;
        std::map<std::string, size_t> offsets;
        hipEvent_t copied = nullptr;       // recorded after the slot's upload
        bool copy_pending = false;
        hipEvent_t fence = nullptr;        // end of the compute that read the slot
        std::vector<hipStream_t> users;    // streams that acquired the slot's current layer
    } slots[2];

    void* resident = nullptr;              // make_resident: every tensor, one allocation
    std::vector<size_t> resident_offsets;  // by tensor position
    std::map<std::string, void*> singles;  // tensors served outside a staged slot

    std::mutex stats_mu;
    long long bytes_streamed = 0;
    double wait_ms = 0, read_ms = 0;
    int staged_layers = 0, skipped_layers = 0;
};

namespace {

int parse_header(qr_model* m) {
    unsigned char head[8];
    const off_t fsize = lseek(m->fd, 0, SEEK_END);
    if (fsize < 8 || pread(m->fd, head, 8, 0) != 8 || memcmp(head, "QWR1", 4) != 0) {
        set_error("%s: not a QuantRunner .qw file", m->path.c_str());
        return QR_ERR_INVALID_ARGUMENT;
    }
    int32_t hlen;
    memcpy(&hlen, head + 4, 4);
    if (hlen <= 0 || 8LL + hlen > fsize) {
        set_error("%s: corrupt header length %d", m->path.c_str(), hlen);
        return QR_ERR_INVALID_ARGUMENT;
    }
    std::string text(static_cast<size_t>(hlen), '\0');
    if (pread(m->fd, &text[0], static_cast<size_t>(hlen), 8) != hlen) {
        set_error("%s: short header read", m->path.c_str());
        return QR_ERR_INVALID_ARGUMENT;
    }
    Json root;
    JsonParser jp{text.data(), text.data() + text.size()};
    if (!jp.value(root) || root.kind != Json::Obj) {
        set_error("%s: header is not a JSON object", m->path.c_str());
        return QR_ERR_INVALID_ARGUMENT;
    }
    // ModelStore.cs:100-106: an explicit data_offset wins; the data start is 64-byte aligned
    long long data_start = 8LL + hlen;
    long long explicit_start;
    if (as_int(root.get("data_offset"), &explicit_start)) data_start = explicit_start;
    if (data_start > LLONG_MAX - 63) {  // the 64-byte rounding would overflow
        set_error("%s: corrupt header (data_offset %lld past the end of the file)", m->path.c_str(), data_start);
        return QR_ERR_INVALID_ARGUMENT;
    }
    data_start = (data_start + 63) & ~63LL;
    if (data_start < 8LL + hlen) {
        set_error("%s: corrupt header (data_offset %lld < header end %lld)", m->path.c_str(), data_start,
                  8LL + hlen);
        return QR_ERR_INVALID_ARGUMENT;
    }
    const Json* ts = root.get("tensors");
    if (!ts || ts->kind != Json::Arr || !root.get("config")) {
        set_error("%s: header lacks the tensors array or the config object", m->path.c_str());
        return QR_ERR_INVALID_ARGUMENT;
    }
    for (const Json& te : ts->arr) {
        const Json* name = te.get("name");
        const Json* dims = te.get("dims");
        long long fmt, off, size;
        if (!name || name->kind != Json::Str || !dims || dims->kind != Json::Arr || !as_int(te.get("format"), &fmt) ||
            !as_int(te.get("offset"), &off) || !as_int(te.get("size"), &size) || off < 0 || size < 0) {
            set_error("%s: malformed tensor entry", m->path.c_str());
            return QR_ERR_INVALID_ARGUMENT;
        }
        Tensor t;
        t.name = name->str;
        for (const Json& d : dims->arr) {
            long long v;
            if (!as_int(&d, &v) || v < 0) {
                set_error("%s: bad dims of tensor %s", m->path.c_str(), t.name.c_str());
                return QR_ERR_INVALID_ARGUMENT;
            }
            t.dims.push_back(v);
        }
        // the reference maps the file and would fault on such a tensor; here it is refused up front
        // (compared without forming data_start + offset + size, which can overflow)
        if (off > fsize - data_start || size > fsize - data_start - off) {
            set_error("%s: tensor %s runs past the end of the file", m->path.c_str(), t.name.c_str());
            return QR_ERR_INVALID_ARGUMENT;
        }
        t.format = static_cast<int>(std::max<long long>(INT_MIN, std::min<long long>(fmt, INT_MAX)));
        t.file_offset = data_start + off;
        t.bytes = size;
        auto it = m->index.find(t.name);
        if (it != m->index.end()) {
            m->tensors[it->second] = std::move(t);  // a repeated name replaces the earlier entry
        } else {
            m->index[t.name] = m->tensors.size();
            m->tensors.push_back(std::move(t));
        }
    }
    return QR_OK;
}

bool read_exact(int fd, void* dst, long long bytes, long long offset) {
    char* d = static_cast<char*>(dst);
    while (bytes > 0) {
        const ssize_t r = pread(fd, d, static_cast<size_t>(std::min<long long>(bytes, 1LL << 30)), offset);
        if (r <= 0) return false;
        d += r;
        bytes -= r;
        offset += r;
    }
    return true;
}

// Reads `chunks` into host + slot_offset with up to `nthreads` threads (the caller's included)
// taking chunks in file order.  `thread_init` runs once on every reading thread before its
// first chunk, `after` on the reading thread after each chunk lands (the staging path queues
// the chunk's upload there); either may be empty.  Returns false on a short read or when
// either callback fails; the other readers stop before their next chunk.
bool parallel_read(int fd, const std::vector<ReadChunk>& chunks, char* host, size_t nthreads,
                   const std::function<bool()>& thread_init, const std::function<bool(const ReadChunk&)>& after) {
    std::atomic<size_t> next{0};
    std::atomic<bool> failed{false};
    auto reader = [&]() {
        if (thread_init && !thread_init()) {
            failed = true;
            return;
        }
        for (size_t i; !failed && (i = next.fetch_add(1)) < chunks.size();) {
            const ReadChunk& c = chunks[i];
            if (!read_exact(fd, host + c.slot_offset, static_cast<long long>(c.bytes), c.file_offset) ||
                (after && !after(c))) {
                failed = true;
                return;
            }
        }
    };
    nthreads = std::max<size_t>(1, std::min(nthreads, chunks.size()));
    std::vector<std::thread> pool;
    for (size_t i = 1; i < nthreads; ++i) {
        try {
            pool.emplace_back(reader);
        } catch (...) {
            break;  // fewer readers
        }
    }
    reader();
    for (auto& t : pool) t.join();
    return !failed;
}

int ensure_device(qr_model* m) {
    if (m->device_ready) return QR_OK;
    QR_HIP(hipGetDevice(&m->device));
    for (auto& s : m->slots) {
        QR_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
        QR_HIP(hipEventCreateWithFlags(&s.copied, hipEventDisableTiming));
        QR_HIP(hipEventCreateWithFlags(&s.fence, hipEventDisableTiming));
    }
    m->device_ready = true;
    return QR_OK;
}

const Tensor* find(const qr_model* m, const char* name) {
    auto it = m->index.find(name);
    return it == m->index.end() ? nullptr : &m->tensors[it->second];
}

// PrefetchPipeline.ReadLayer (PrefetchPipeline.cs:111-166) on the slot's worker thread: the
// layer's tensors (prefix "l<layer>.", all tensors for a negative layer; names ending in "norm"
// or "router" stay outside) are read into the pinned buffer and uploaded on the slot's copy
// stream.  Over budget or failed: the slot stays unstaged and Acquire serves the tensors one by
// one, as the reference falls back to the mmap.
void read_layer(qr_model* m, qr_model::Slot* s, int layer) {
    const auto t0 = std::chrono::steady_clock::now();
    struct Tick {
        qr_model* m;
        std::chrono::steady_clock::time_point t0;
        ~Tick() {
            std::lock_guard<std::mutex> g(m->stats_mu);
            m->read_ms += ms_since(t0);
        }
    } tick{m, t0};
    if (hipSetDevice(m->device) != hipSuccess) return;
    const std::string prefix = layer < 0 ? std::string() : "l" + std::to_string(layer) + ".";
    std::vector<const Tensor*> list;
    long long total = 0;
    size_t padded = 0;
    for (const Tensor& t : m->tensors) {
        if (!prefix.empty() && t.name.compare(0, prefix.size(), prefix) != 0) continue;
        if (ends_with(t.name, "norm") || ends_with(t.name, "router")) continue;
        list.push_back(&t);
        total += t.bytes;
        padded += align_up(static_cast<size_t>(t.bytes));
    }
    if (total == 0 || total > m->budget) {
        std::lock_guard<std::mutex> g(m->stats_mu);
        ++m->skipped_layers;
        return;
    }
    // the pinned buffer is rewritten only after its previous upload finished
    if (s->copy_pending && hipEventSynchronize(s->copied) != hipSuccess) return;
    s->copy_pending = false;
    if (s->pinned_cap < padded) {
        if (s->pinned) (void)hipHostFree(s->pinned);
        s->pinned = nullptr;
        s->pinned_cap = 0;
        if (hipHostMalloc(&s->pinned, padded, hipHostMallocDefault) != hipSuccess) return;
        s->pinned_cap = padded;
    }
    if (s->dev_cap < padded) {
        // the old slot may still be read by compute fenced on the copy stream
        if (hipStreamSynchronize(s->stream) != hipSuccess) return;
        if (s->dev) (void)hipFree(s->dev);
        s->dev = nullptr;
        s->dev_cap = 0;
        if (hipMalloc(&s->dev, padded) != hipSuccess) return;
        s->dev_cap = padded;
    }
    // Chunks of at most kReadChunk bytes, never across a tensor: reader threads take them in
    // file order, read each into the pinned buffer and queue its upload at once, so the file
    // reads run in parallel and overlap the host-to-device copies.
    std::map<std::string, size_t> offsets;
    std::vector<ReadChunk> chunks;
    size_t off = 0;
    for (const Tensor* t : list) {
        offsets[t->name] = off;
        const long long step = static_cast<long long>(m->read_chunk);
        for (long long c = 0; c < t->bytes; c += step)
            chunks.push_back({off + static_cast<size_t>(c), t->file_offset + c,
                              static_cast<size_t>(std::min<long long>(step, t->bytes - c))});
        off += align_up(static_cast<size_t>(t->bytes));
    }
    std::atomic<bool> queued{false};
    char* pinned = static_cast<char*>(s->pinned);
    const bool ok = parallel_read(
        m->fd, chunks, pinned, m->read_threads, [m]() { return hipSetDevice(m->device) == hipSuccess; },
        [&](const ReadChunk& c) {
            if (hipMemcpyAsync(static_cast<char*>(s->dev) + c.slot_offset, pinned + c.slot_offset, c.bytes,
                               hipMemcpyHostToDevice, s->stream) != hipSuccess)
                return false;
            queued = true;
            return true;
        });
    // stream order puts the uploads after the fences Begin placed on this copy stream
    if (queued) {
        if (hipEventRecord(s->copied, s->stream) != hipSuccess) {
            (void)hipStreamSynchronize(s->stream);
            return;
        }
        s->copy_pending = true;
    }
    if (!ok) return;
    s->offsets.swap(offsets);
    s->staged = true;
    std::lock_guard<std::mutex> g(m->stats_mu);
    m->bytes_streamed += total;
    ++m->staged_layers;
}

void join(qr_model::Slot& s) {
    if (s.task.joinable()) s.task.join();
}

// PrefetchPipeline.cs:87-92: time the caller spends waiting on a read
void join_timed(qr_model* m, qr_model::Slot& s) {
    if (!s.task.joinable()) return;
    const auto t0 = std::chrono::steady_clock::now();
    s.task.join();
    std::lock_guard<std::mutex> g(m->stats_mu);
    m->wait_ms += ms_since(t0);
}

// A tensor outside a staged slot (norms, routers, over-budget layers, pipeline off): uploaded
// once and kept, as the reference's mmap view of it stays valid until Dispose.
int single(qr_model* m, const Tensor& t, const void** out) {
    auto it = m->singles.find(t.name);
    if (it != m->singles.end()) {
        *out = it->second;
        return QR_OK;
    }
    std::vector<char> host(static_cast<size_t>(t.bytes));
    if (t.bytes && !read_exact(m->fd, host.data(), t.bytes, t.file_offset)) {
        set_error("%s: short read of tensor %s", m->path.c_str(), t.name.c_str());
        return QR_ERR_INVALID_ARGUMENT;
    }
    void* d = nullptr;
    QR_HIP(hipMalloc(&d, std::max(align_up(static_cast<size_t>(t.bytes)), kAlign)));
    if (t.bytes) {
        const hipError_t e = hipMemcpy(d, host.data(), static_cast<size_t>(t.bytes), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            QR_HIP(e);
        }
    }
    m->singles[t.name] = d;
    *out = d;
    return QR_OK;
}

#define QR_CHECK_MODEL(m) QR_CHECK_ARG((m) != nullptr, "null qr_model handle")

}  // namespace

extern "C" {

int qr_model_open(qr_model** out, const char* path) {
    clear_error();
    QR_CHECK_ARG(out != nullptr && path != nullptr, "null output or path");
    *out = nullptr;
    qr_model* m = new (std::nothrow) qr_model();
    if (!m) {
        set_error("host allocation of the handle failed");
        return QR_ERR_OUT_OF_MEMORY;
    }
    m->path = path;
    m->read_threads = env_size("QR_PREFETCH_READERS", kReadThreads, 1, 64);
    m->read_chunk = env_size("QR_PREFETCH_CHUNK_MB", kReadChunk >> 20, 1, 256) << 20;
    m->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (m->fd < 0) {
        set_error("cannot open %s", path);
        delete m;
        return QR_ERR_INVALID_ARGUMENT;
    }
    const int st = parse_header(m);
    if (st != QR_OK) {
        close(m->fd);
        delete m;
        return st;
    }
    *out = m;
    return QR_OK;
}

int qr_model_close(qr_model* m) {
    clear_error();
    if (!m) return QR_OK;
    for (auto& s : m->slots) join(s);
    if (m->device_ready) {
        DeviceGuard dg(m->device);
        // uploads, and launches that may still read a slot on streams the caller owns (and may
        // have destroyed since): wait for the whole device
        (void)hipDeviceSynchronize();
        for (auto& s : m->slots) {
            if (s.pinned) (void)hipHostFree(s.pinned);
            if (s.dev) (void)hipFree(s.dev);
            (void)hipEventDestroy(s.copied);
            (void)hipEventDestroy(s.fence);
            (void)hipStreamDestroy(s.stream);
        }
        if (m->resident) (void)hipFree(m->resident);
        for (auto& kv : m->singles) (void)hipFree(kv.second);
    }
    if (m->fd >= 0) close(m->fd);
    delete m;
    return QR_OK;
}

int qr_model_tensor_count(const qr_model* m, int* count) {
    clear_error();
    QR_CHECK_MODEL(m);
    QR_CHECK_ARG(count != nullptr, "null output");
    *count = static_cast<int>(m->tensors.size());
    return QR_OK;
}

int qr_model_tensor_name(const qr_model* m, int i, char* buf, int buf_len) {
    clear_error();
    QR_CHECK_MODEL(m);
    QR_CHECK_ARG(i >= 0 && static_cast<size_t>(i) < m->tensors.size(), "tensor index %d out of range [0, %zu)", i,
                 m->tensors.size());
    const std::string& n = m->tensors[static_cast<size_t>(i)].name;
    QR_CHECK_ARG(buf != nullptr && buf_len > static_cast<int>(n.size()), "name buffer needs %zu bytes",
                 n.size() + 1);
    memcpy(buf, n.c_str(), n.size() + 1);
    return QR_OK;
}

int qr_model_tensor_info(const qr_model* m, const char* name, int* format, int* ndims, long long* dims,
                         int dims_cap, long long* bytes) {
    clear_error();
    QR_CHECK_MODEL(m);
    QR_CHECK_ARG(name != nullptr, "null tensor name");
    const Tensor* t = find(m, name);
    QR_CHECK_ARG(t != nullptr, "tensor '%s' not found in %s", name, m->path.c_str());
    QR_CHECK_ARG(dims == nullptr || dims_cap >= static_cast<int>(t->dims.size()), "tensor '%s' has %zu dims", name,
                 t->dims.size());
    if (format) *format = t->format;
    if (ndims) *ndims = static_cast<int>(t->dims.size());
    if (dims)
        for (size_t i = 0; i < t->dims.size(); ++i) dims[i] = t->dims[i];
    if (bytes) *bytes = t->bytes;
    return QR_OK;
}

int qr_model_read(const qr_model* m, const char* name, void* dst, long long dst_bytes) {
    clear_error();
    QR_CHECK_MODEL(m);
    QR_CHECK_ARG(name != nullptr, "null tensor name");
    const Tensor* t = find(m, name);
    QR_CHECK_ARG(t != nullptr, "tensor '%s' not found in %s", name, m->path.c_str());
    QR_CHECK_ARG(dst != nullptr || t->bytes == 0, "null destination");
    QR_CHECK_ARG(dst_bytes >= t->bytes, "tensor '%s' needs %lld bytes, buffer holds %lld", name, t->bytes, dst_bytes);
    // large tensors are read in chunks by the prefetch readers, in parallel
    std::vector<ReadChunk> chunks;
    const long long step = static_cast<long long>(m->read_chunk);
    for (long long c = 0; c < t->bytes; c += step)
        chunks.push_back({static_cast<size_t>(c), t->file_offset + c, static_cast<size_t>(std::min<long long>(step, t->bytes - c))});
    if (!parallel_read(m->fd, chunks, static_cast<char*>(dst), m->read_threads, nullptr, nullptr)) {
        set_error("%s: short read of tensor %s", m->path.c_str(), name);
        return QR_ERR_INVALID_ARGUMENT;
    }
    return QR_OK;
}

int qr_model_set_prefetch(qr_model* m, long long budget_bytes) {
    clear_error();
    QR_CHECK_MODEL(m);
    QR_CHECK_ARG(budget_bytes >= 0, "negative prefetch budget %lld", budget_bytes);
    for (auto& s : m->slots) {
        join(s);
        s.for_layer = INT_MIN;
        s.staged = false;
    }
    m->budget = budget_bytes;
    return QR_OK;
}

int qr_model_begin(qr_model* m, int layer) {
    clear_error();
    QR_CHECK_MODEL(m);
    if (m->budget <= 0 || m->resident) return QR_OK;
    QR_TRY(ensure_device(m));
    DeviceGuard dg(m->device);
    qr_model::Slot& s = m->slots[layer & 1];
    join(s);  // PrefetchPipeline.cs:69-70: the previous read into this slot
    // Work enqueued so far on every stream that acquired the slot's previous layer may still read
    // the slot: the next upload into it waits for that work, on the GPU.
    for (hipStream_t u : s.users) {
        QR_HIP(hipEventRecord(s.fence, u));
        QR_HIP(hipStreamWaitEvent(s.stream, s.fence, 0));
    }
    s.users.clear();
    s.for_layer = layer;
    s.staged = false;
    s.offsets.clear();
    try {
        s.task = std::thread(read_layer, m, &s, layer);
    } catch (...) {
        s.for_layer = INT_MIN;
        set_error("cannot start the prefetch thread");
        return QR_ERR_OUT_OF_MEMORY;
    }
    return QR_OK;
}

int qr_model_acquire(qr_model* m, const char* name, int layer, void* stream, const void** dev_ptr) {
    clear_error();
    QR_CHECK_MODEL(m);
    QR_CHECK_ARG(name != nullptr && dev_ptr != nullptr, "null name or output");
    *dev_ptr = nullptr;
    const Tensor* t = find(m, name);
    QR_CHECK_ARG(t != nullptr, "tensor '%s' not found in %s", name, m->path.c_str());
    QR_TRY(ensure_device(m));
    DeviceGuard dg(m->device);
    if (m->resident) {
        *dev_ptr = static_cast<char*>(m->resident) + m->resident_offsets[m->index.at(name)];
        return QR_OK;
    }
    qr_model::Slot& s = m->slots[layer & 1];
    if (m->budget > 0 && s.for_layer == layer) {
        join_timed(m, s);
        auto o = s.staged ? s.offsets.find(name) : s.offsets.end();
        if (o != s.offsets.end()) {
            const hipStream_t st = static_cast<hipStream_t>(stream);
            QR_HIP(hipStreamWaitEvent(st, s.copied, 0));
            bool known = false;
            for (hipStream_t u : s.users) known |= u == st;
            if (!known) s.users.push_back(st);
            *dev_ptr = static_cast<char*>(s.dev) + o->second;
            return QR_OK;
        }
    }
    return single(m, *t, dev_ptr);
}

int qr_model_release(qr_model* m, int layer, void* stream) {
    clear_error();
    QR_CHECK_MODEL(m);
    if (!m->device_ready || m->resident) return QR_OK;
    qr_model::Slot& s = m->slots[layer & 1];
    if (s.for_layer != layer) return QR_OK;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    for (size_t i = 0; i < s.users.size(); ++i) {
        if (s.users[i] != st) continue;
        DeviceGuard dg(m->device);
        QR_HIP(hipEventRecord(s.fence, st));
        QR_HIP(hipStreamWaitEvent(s.stream, s.fence, 0));
        s.users.erase(s.users.begin() + static_cast<long>(i));
        break;
    }
    return QR_OK;
}

int qr_model_wait_layer(qr_model* m, int layer) {
    clear_error();
    QR_CHECK_MODEL(m);
    qr_model::Slot& s = m->slots[layer & 1];
    if (s.for_layer == layer) join_timed(m, s);
    return QR_OK;
}

int qr_model_make_resident(qr_model* m) {
    clear_error();
    QR_CHECK_MODEL(m);
    if (m->resident) return QR_OK;
    QR_TRY(ensure_device(m));
    DeviceGuard dg(m->device);
    for (auto& s : m->slots) join(s);
    size_t total = 0;
    std::vector<size_t> offsets;
    for (const Tensor& t : m->tensors) {
        offsets.push_back(total);
        total += align_up(static_cast<size_t>(t.bytes));
    }
    void* dev = nullptr;
    QR_HIP(hipMalloc(&dev, std::max(total, kAlign)));
    // file -> two pinned chunks -> HBM, the read of one chunk overlapping the upload of the other
    const size_t chunk = 64u << 20;
    hipStream_t cs = m->slots[0].stream;
    void* pinned[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    int st = QR_OK;
    for (int i = 0; i < 2 && st == QR_OK; ++i)
        if (hipHostMalloc(&pinned[i], chunk, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) {
            set_error("pinned staging allocation of %zu bytes failed", chunk);
            st = QR_ERR_OUT_OF_MEMORY;
        }
    int k = 0;
    long long streamed = 0;
    for (size_t ti = 0; ti < m->tensors.size() && st == QR_OK; ++ti) {
        const Tensor& t = m->tensors[ti];
        long long left = t.bytes, src = t.file_offset;
        size_t dst = offsets[ti];
        while (left > 0) {
            const size_t n = static_cast<size_t>(std::min<long long>(left, static_cast<long long>(chunk)));
            if (used[k] && hipEventSynchronize(done[k]) != hipSuccess) {
                set_error("resident upload: event wait failed");
                st = QR_ERR_HIP;
                break;
            }
            if (!read_exact(m->fd, pinned[k], static_cast<long long>(n), src)) {
                set_error("%s: short read of tensor %s", m->path.c_str(), t.name.c_str());
                st = QR_ERR_INVALID_ARGUMENT;
                break;
            }
            if (hipMemcpyAsync(static_cast<char*>(dev) + dst, pinned[k], n, hipMemcpyHostToDevice, cs) != hipSuccess ||
                hipEventRecord(done[k], cs) != hipSuccess) {
                set_error("resident upload: copy failed");
                st = QR_ERR_HIP;
                break;
            }
            used[k] = true;
            k ^= 1;
            left -= static_cast<long long>(n);
            src += static_cast<long long>(n);
            dst += n;
        }
        streamed += t.bytes;
    }
    if (hipStreamSynchronize(cs) != hipSuccess && st == QR_OK) {
        set_error("resident upload: stream synchronize failed");
        st = QR_ERR_HIP;
    }
    for (int i = 0; i < 2; ++i) {
        if (pinned[i]) (void)hipHostFree(pinned[i]);
        if (done[i]) (void)hipEventDestroy(done[i]);
    }
    if (st != QR_OK) {
        (void)hipFree(dev);
        return st;
    }
    m->resident = dev;
    m->resident_offsets.swap(offsets);
    std::lock_guard<std::mutex> g(m->stats_mu);
    m->bytes_streamed += streamed;
    return QR_OK;
}

int qr_model_stats(qr_model* m, long long* bytes_streamed, double* wait_ms, double* read_ms, int* staged_layers,
                   int* skipped_layers) {
    clear_error();
    QR_CHECK_MODEL(m);
    std::lock_guard<std::mutex> g(m->stats_mu);
    if (bytes_streamed) *bytes_streamed = m->bytes_streamed;
    if (wait_ms) *wait_ms = m->wait_ms;
    if (read_ms) *read_ms = m->read_ms;
    if (staged_layers) *staged_layers = m->staged_layers;
    if (skipped_layers) *skipped_layers = m->skipped_layers;
    return QR_OK;
}

}  // extern "C"
