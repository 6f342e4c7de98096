// qr_store.cpp -- HBM page pool, device page tables, error plumbing.
#include "qr_store.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <string>

namespace qr {

// ---------------------------------------------------------------- errors
namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

const char* last_error() { return g_last_error.c_str(); }

// ---------------------------------------------------------------- DevBuf
DevBuf::~DevBuf() {
    if (ptr_) (void)hipFree(ptr_);
    for (void* r : retired_) (void)hipFree(r);
}

int DevBuf::ensure(size_t bytes, bool zero) {
    if (bytes <= size_) return QR_OK;
    if (ptr_ && keep_retired_) {
        retired_.push_back(ptr_);  // a captured graph may still use it: freed with the buffer
        ptr_ = nullptr;
        size_ = 0;
    } else if (ptr_) {
        QR_HIP(hipDeviceSynchronize());
        QR_HIP(hipFree(ptr_));
        ptr_ = nullptr;
        size_ = 0;
    }
    size_t want = std::max(bytes, size_ * 2);
    want = (want + 255) & ~static_cast<size_t>(255);
    QR_HIP(hipMalloc(&ptr_, want));
    size_ = want;
    if (zero) QR_HIP(hipMemset(ptr_, 0, want));
    return QR_OK;
}

// ---------------------------------------------------------------- PagedStore
PagedStore::~PagedStore() {
    if (pool_) (void)hipFree(pool_);
    if (pt_dev_) (void)hipFree(pt_dev_);
    if (state_dev_) (void)hipFree(state_dev_);
}

int PagedStore::init(const PageGeom& geom, int dtype, int layers, int seqs, int max_seq) {
    geom_ = geom;
    dtype_ = dtype;
    layers_ = layers;
    seqs_ = seqs;
    max_pages_ = (max_seq + kPageTokens - 1) / kPageTokens;
    const size_t entries = static_cast<size_t>(seqs) * layers * max_pages_;
    pt_host_.assign(entries, 0);
    held_.assign(static_cast<size_t>(seqs) * layers, 0);
    QR_HIP(hipMalloc(&pt_dev_, std::max<size_t>(entries, 1) * sizeof(int)));
    QR_HIP(hipMemset(pt_dev_, 0, std::max<size_t>(entries, 1) * sizeof(int)));
    state_host_.assign(2 + static_cast<size_t>(seqs) * layers + seqs, 0);
    QR_HIP(hipMalloc(&state_dev_, state_host_.size() * sizeof(int)));
    QR_HIP(hipMemset(state_dev_, 0, state_host_.size() * sizeof(int)));
    return QR_OK;
}

int PagedStore::pull(std::vector<int>& seq_len) {
    if (!device_ahead()) return QR_OK;
    QR_HIP(hipDeviceSynchronize());  // the device-side appends were enqueued on caller streams
    QR_HIP(hipMemcpy(state_host_.data(), state_dev_, state_host_.size() * sizeof(int), hipMemcpyDeviceToHost));
    device_ahead_ = false;
    pages_used_ = state_host_[0];
    for (size_t i = 0; i < held_.size(); ++i) held_[i] = state_host_[2 + i];
    for (int s = 0; s < seqs_; ++s) seq_len[s] = state_host_[seq_index(s)];
    const int err = state_host_[1];
    if (err) {
        QR_HIP(hipMemset(state_dev_ + 1, 0, sizeof(int)));
        set_error("a device-side append failed: %s%s", (err & 1) ? "the page pool was full (reserve more pages) " : "",
                  (err & 2) ? "a position was outside [0, max_seq)" : "");
        return (err & 1) ? QR_ERR_OUT_OF_MEMORY : QR_ERR_OUT_OF_RANGE;
    }
    return QR_OK;
}

int PagedStore::push(const std::vector<int>& seq_len, hipStream_t stream) {
    state_host_[0] = static_cast<int>(pages_used_);
    state_host_[1] = 0;
    for (size_t i = 0; i < held_.size(); ++i) state_host_[2 + i] = held_[i];
    for (int s = 0; s < seqs_; ++s) state_host_[seq_index(s)] = seq_len[s];
    QR_HIP(hipMemcpyAsync(state_dev_, state_host_.data(), state_host_.size() * sizeof(int), hipMemcpyHostToDevice, stream));
    return QR_OK;
}

int PagedStore::grow(long long min_pages) {
    if (min_pages <= pool_cap_) return QR_OK;
    if (frozen_) {
        set_error("the page pool holds %lld pages and cannot grow to %lld: a captured graph uses its address "
                  "(reserve the pages before capturing)", pool_cap_, min_pages);
        return QR_ERR_OUT_OF_MEMORY;
    }
    const long long cap = std::max(min_pages, std::max(pool_cap_ * 2, 16LL));
    const size_t pb = static_cast<size_t>(page_bytes());
    char* fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, cap * pb);
    if (e != hipSuccess && cap > min_pages) {
        (void)hipGetLastError();
        e = hipMalloc(&fresh, min_pages * pb);  // doubling failed: take exactly what is needed
        if (e == hipSuccess) return grow_done(fresh, min_pages, pb);
    }
    if (e != hipSuccess) {
        set_error("page pool growth to %lld pages (%zu bytes each) failed: %s", cap, pb, hipGetErrorString(e));
        return QR_ERR_OUT_OF_MEMORY;
    }
    return grow_done(fresh, cap, pb);
}

int PagedStore::grow_done(char* fresh, long long cap, size_t pb) {
    QR_HIP(hipMemset(fresh + pool_cap_ * pb, 0, (cap - pool_cap_) * pb));
    if (pool_) {
        QR_HIP(hipDeviceSynchronize());  // kernels on any stream may still read the old pool
        QR_HIP(hipMemcpy(fresh, pool_, pool_cap_ * pb, hipMemcpyDeviceToDevice));
        QR_HIP(hipFree(pool_));
    }
    QR_HIP(hipDeviceSynchronize());
    pool_ = fresh;
    pool_cap_ = cap;
    return QR_OK;
}

int PagedStore::reserve(int pages) {
    QR_CHECK_ARG(pages >= 0, "reserve: pages must be >= 0 (got %d)", pages);
    return grow(pages);
}

int PagedStore::ensure(int seq, int layer, int tokens, hipStream_t stream) {
    const int need = (tokens + kPageTokens - 1) / kPageTokens;
    int& h = held_[static_cast<size_t>(seq) * layers_ + layer];
    if (need <= h) return QR_OK;
    const long long add = need - h;
    QR_TRY(grow(pages_used_ + add));
    const int row = pt_offset(seq, layer);
    for (int i = h; i < need; ++i) pt_host_[row + i] = static_cast<int>(pages_used_++);
    QR_HIP(hipMemcpyAsync(pt_dev_ + row + h, pt_host_.data() + row + h, add * sizeof(int),
                          hipMemcpyHostToDevice, stream));
    h = need;
    return QR_OK;
}

}  // namespace qr
