// Device workspaces of the f32 entry points: quantised activations, padded
// copies, split-K planes and the MLP's intermediate rows.
//
// Ownership rule: a buffer belongs to one (device, stream, host thread,
// kind).  A host thread's calls are sequential and its launches on one
// stream are ordered, so reusing that buffer from call to call is race-free.
// Two threads sharing a stream get different buffers, so their launches may
// interleave on the stream without one call reading the other's rows (the
// reference's `forward(&self)` is shared across threads through Arc).
//
// Buffers are never freed while the library runs: a buffer that has to grow
// is retired (kept) and a larger one takes its place, because launches
// already queued, or a HIP graph captured earlier, may still use the old
// address.  Retired and live buffers are freed only by release_all() (the
// caller's explicit xt_workspace_release, or process teardown).  Growth
// doubles the capacity, so the retired buffers together stay below the live
// one.
//
// A host thread that ends hands its buffers to a pool (thread_exit, called
// from a thread_local guard in the library).  A (device, stream, thread,
// kind) that needs its first buffer adopts a pooled one of the same device
// and kind that is large enough, after one device synchronize (the ended
// thread's launches may still be queued), instead of allocating.  So a host
// that spawns short-lived threads holds at most as many buffers per kind as
// it has threads calling at the same time, not one per thread ever started.
//
// While the stream is being captured into a graph the table never allocates
// (no allocation, memset or synchronisation may enter a capture): a request
// that fits the existing buffer is served, one that would grow it fails with
// kCapture and a message.
//
// The HIP calls are behind a function table so the same logic runs in a CPU
// test with a fake backend.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

namespace xt {

struct WsBackend {
    // each returns 0 on success, non-zero (a backend error code) otherwise
    int (*current_device)(int* dev);
    int (*alloc)(void** p, size_t bytes);
    int (*free_)(void* p);
    int (*is_capturing)(void* stream, bool* capturing);
    int (*zero)(void* p, size_t bytes, void* stream);  // stream-ordered clear
    int (*device_sync)();
    const char* (*error_string)(int code);
};

class WorkspaceTable {
public:
    enum Status { kOk = 0, kBackend = 1, kNoMem = 2, kCapture = 3 };

    explicit WorkspaceTable(const WsBackend& b) : b_(b) {}

    // A buffer of at least `bytes` for this (device, stream, calling thread,
    // kind).  zero_new: clear a newly allocated buffer on the stream (split-K
    // counters must start at zero).
    int get(void* stream, size_t bytes, int kind, bool zero_new, void** out, std::string* err) {
        int dev = 0;
        if (int e = b_.current_device(&dev)) return backend_fail(e, "get device", err);
        std::lock_guard<std::mutex> lk(mu_);
        Entry& w = table_[Key(dev, stream, std::this_thread::get_id(), kind)];
        if (w.ptr && w.cap >= bytes && !w.stale) {
            *out = w.ptr;
            return kOk;
        }
        bool cap_active = false;
        if (int e = b_.is_capturing(stream, &cap_active)) return backend_fail(e, "capture query", err);
        if (cap_active) {
            *err = "workspace of " + std::to_string(bytes) +
                   " bytes would have to be allocated during graph capture; make one eager call "
                   "of the largest shape on this stream and thread before capturing";
            return kCapture;
        }
        if (!w.ptr) {  // a first buffer for this key: adopt a pooled one
            for (size_t i = 0; i < pool_.size(); ++i) {
                const Pooled& pb = pool_[i];
                if (pb.dev != dev || pb.kind != kind || pb.stale || pb.cap < bytes) continue;
                if (int e = b_.device_sync()) return backend_fail(e, "device synchronize", err);
                w.ptr = pb.ptr;
                w.cap = pb.cap;
                w.stale = false;
                pool_.erase(pool_.begin() + (ptrdiff_t)i);
                *out = w.ptr;
                return kOk;
            }
        }
        size_t cap = w.cap * 2;
        if (cap < bytes) cap = bytes;
        if (cap < kMinBytes) cap = kMinBytes;
        cap = (cap + 4095) / 4096 * 4096;
        void* p = nullptr;
        if (int e = b_.alloc(&p, cap)) {
            *err = std::string("workspace allocation of ") + std::to_string(cap) +
                   " bytes: " + b_.error_string(e);
            return kNoMem;
        }
        if (zero_new) {
            if (int e = b_.zero(p, cap, stream)) {
                (void)b_.free_(p);
                return backend_fail(e, "workspace clear", err);
            }
        }
        if (w.ptr) retired_.push_back(w.ptr);  // queued work or a graph may still use it
        w.ptr = p;
        w.cap = cap;
        w.stale = false;
        *out = p;
        return kOk;
    }

    // Make every buffer of `kind` be replaced on its next use (the split-K
    // counter region moved).
    void mark_stale(int kind) {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto& kv : table_)
            if (std::get<3>(kv.first) == kind) kv.second.stale = true;
        for (Pooled& pb : pool_)
            if (pb.kind == kind) pb.stale = true;
    }

    // The calling thread `id` ends: its buffers go to the pool.
    void thread_exit(std::thread::id id) {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto it = table_.begin(); it != table_.end();) {
            if (std::get<2>(it->first) == id) {
                if (it->second.ptr)
                    pool_.push_back(Pooled{std::get<0>(it->first), std::get<3>(it->first), it->second.ptr,
                                           it->second.cap, it->second.stale});
                it = table_.erase(it);
            } else {
                ++it;
            }
        }
    }

    // Wait for the device, then free every buffer (live and retired).  The
    // caller guarantees that no graph using them will be replayed.
    int release_all(std::string* err) {
        std::lock_guard<std::mutex> lk(mu_);
        if (int e = b_.device_sync()) return backend_fail(e, "device synchronize", err);
        int rc = kOk;
        for (auto& kv : table_)
            if (kv.second.ptr && b_.free_(kv.second.ptr)) rc = kBackend;
        for (void* p : retired_)
            if (b_.free_(p)) rc = kBackend;
        for (const Pooled& pb : pool_)
            if (b_.free_(pb.ptr)) rc = kBackend;
        table_.clear();
        retired_.clear();
        pool_.clear();
        if (rc) *err = "workspace free failed";
        return rc;
    }

    size_t live_count() {
        std::lock_guard<std::mutex> lk(mu_);
        size_t n = 0;
        for (auto& kv : table_) n += kv.second.ptr != nullptr;
        return n;
    }
    size_t retired_count() {
        std::lock_guard<std::mutex> lk(mu_);
        return retired_.size();
    }
    size_t pooled_count() {
        std::lock_guard<std::mutex> lk(mu_);
        return pool_.size();
    }

    static constexpr size_t kMinBytes = (size_t)1 << 20;

private:
    struct Entry {
        void* ptr = nullptr;
        size_t cap = 0;
        bool stale = false;
    };
    typedef std::tuple<int, void*, std::thread::id, int> Key;
    struct Pooled {
        int dev, kind;
        void* ptr;
        size_t cap;
        bool stale;
    };

    int backend_fail(int e, const char* what, std::string* err) {
        *err = std::string(what) + ": " + b_.error_string(e);
        return kBackend;
    }

    WsBackend b_;
    std::mutex mu_;
    std::map<Key, Entry> table_;
    std::vector<void*> retired_;
    std::vector<Pooled> pool_;  // buffers of threads that have ended
};

}  // namespace xt
