// qr_store.hpp -- HBM page pool + device page tables shared by the KV and MLA caches.
#pragma once

#include <vector>

#include "qr_kernels.hpp"

namespace qr {

// Makes the handle's device current for the duration of a call.
class DeviceGuard {
public:
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        if (prev_ != device) ok_ = hipSetDevice(device) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
    }
    bool ok() const { return ok_; }

private:
    int prev_ = -1;
    bool ok_ = true;
};

// Growable device buffer.  Growing waits for the device to go idle first,
// because work enqueued on any stream may still read the old allocation.  Once a
// captured graph holds the buffer's address (keep_retired), growing no longer frees
// the old allocation: it stays valid for the graph's replays until the buffer is
// destroyed.
class DevBuf {
public:
    ~DevBuf();
    // zero: a new allocation is zero-filled before it is returned
    int ensure(size_t bytes, bool zero = false);
    void keep_retired() { keep_retired_ = true; }
    void* get() const { return ptr_; }
    size_t size() const { return size_; }

private:
    void* ptr_ = nullptr;
    size_t size_ = 0;
    bool keep_retired_ = false;
    std::vector<void*> retired_;
};

// Page pool of one cache: `seqs` sequences x `layers` layers, each with a row
// of `max_pages` page-table entries.  A page is allocated when any of its
// positions is first appended (the intended behaviour of PagedKvCache.Ensure,
// PagedKvCache.cs:41-60; every page up to the appended one is allocated) and
// is zero-filled at allocation, as a fresh managed array is.
class PagedStore {
public:
    ~PagedStore();
    int init(const PageGeom& geom, int dtype, int layers, int seqs, int max_seq);
    // Makes positions 0..tokens-1 of (seq, layer) resident; uploads new page-table entries.
    int ensure(int seq, int layer, int tokens, hipStream_t stream);
    int reserve(int pages);
    // A captured graph holds the pool's address: from now on the pool never moves, and
    // growing past its capacity is an error (the caller reserves pages before capturing).
    void freeze() { frozen_ = true; }
    bool frozen() const { return frozen_; }

    int pages_held(int seq, int layer) const { return held_[static_cast<size_t>(seq) * layers_ + layer]; }
    bool resident(int seq, int layer, int pos) const {
        return static_cast<long long>(pages_held(seq, layer)) * kPageTokens > pos;
    }
    int pt_offset(int seq, int layer) const { return (seq * layers_ + layer) * max_pages_; }
    const int* page_table_dev() const { return pt_dev_; }
    void* pool() const { return pool_; }
    const PageGeom& geom() const { return geom_; }
    int dtype() const { return dtype_; }
    long long page_bytes() const { return geom_.page_elems() * dtype_size(dtype_); }
    long long bytes_used() const { return pages_used_ * page_bytes(); }
    int max_pages() const { return max_pages_; }
    long long capacity() const { return pool_cap_; }

    // Device copy of the page accounting, for appends whose position is read on the
    // device (page_claim_kernel): [0] pages handed out, [1] error bits, then the held
    // count of every (seq, layer), then SeqLen of every sequence.  The host copy is
    // authoritative until a device-side append is enqueued (mark_device_ahead); the
    // next host-side call then waits for the device and reads it back (pull).
    int* state_dev() const { return state_dev_; }
    int held_index(int seq, int layer) const { return 2 + seq * layers_ + layer; }
    int seq_index(int seq) const { return 2 + seqs_ * layers_ + seq; }
    void mark_device_ahead() { device_ahead_ = true; }
    // A device-side append captured into a graph may be replayed at any time, so from then on
    // every host-side call reads the device accounting back first.
    void mark_replayable() { replayable_ = true; }
    bool device_ahead() const { return device_ahead_ || replayable_; }
    // Waits for the device, takes pages used and held counts from its copy and stores
    // SeqLen into seq_len; device error bits become an error return (and are cleared).
    int pull(std::vector<int>& seq_len);
    // Writes the host accounting and seq_len to the device copy (on `stream`).
    int push(const std::vector<int>& seq_len, hipStream_t stream);

private:
    int grow(long long min_pages);
    int grow_done(char* fresh, long long cap, size_t page_bytes);

    PageGeom geom_{};
    int dtype_ = QR_DTYPE_F32;
    int layers_ = 0, seqs_ = 0, max_pages_ = 0;
    char* pool_ = nullptr;
    long long pool_cap_ = 0;   // pages allocated in the pool
    long long pages_used_ = 0; // pages handed out
    std::vector<int> pt_host_;
    int* pt_dev_ = nullptr;
    std::vector<int> held_;
    int* state_dev_ = nullptr;
    std::vector<int> state_host_;
    bool device_ahead_ = false;
    bool replayable_ = false;
    bool frozen_ = false;
};

}  // namespace qr
