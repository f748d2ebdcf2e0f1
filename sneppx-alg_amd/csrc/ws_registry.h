// ws_registry.h - the library's scratch workspaces, kept per
// (device, stream, slot) for each host thread, with no device calls of its
// own: allocation and stream-ordered release go through the two callbacks
// given to snx_ws::init (HIP's stream-ordered pool in runtime.hip, malloc in
// the CPU test of this logic).
//
// Rules:
//  * A thread looks its buffers up in a thread_local table (a few entries:
//    one per stream and slot it has used), without a lock.  Two threads never
//    share a buffer, even on one stream: a call's kernels (a split-K partial
//    pass and its reduction, say) may then interleave with another thread's
//    on that stream without reading each other's scratch.
//  * A larger request takes a new buffer and releases the old one ordered on
//    the same stream, after the work already queued there.
//  * When a thread ends, its table's destructor moves its buffers to a shared
//    list of orphans (no device call: the stream may already be gone at that
//    point, or the runtime torn down at process exit).  The next thread that
//    needs the same (device, stream, slot) adopts an orphan instead of
//    allocating: its last use was queued on that stream by a thread that has
//    ended, so work queued there afterwards is ordered behind it.  A pool of
//    short-lived request threads therefore holds as many buffers per
//    (stream, slot) as it has threads alive at once, not as it ever had.
//  * release_stream(stream) frees the calling thread's buffers and every
//    orphan on `stream`, for a caller about to destroy that stream.
#ifndef SNX_WS_REGISTRY_H
#define SNX_WS_REGISTRY_H

#include <atomic>
#include <cstddef>
#include <mutex>
#include <vector>

namespace snx_ws {

// alloc: a buffer of `bytes` usable by work queued on `stream` (zero-filled
// on `stream` when `zeroed`), nullptr on failure.  release: frees `p` after
// the work already queued on `stream`.
using AllocFn = void* (*)(size_t bytes, void* stream, bool zeroed);
using ReleaseFn = void (*)(void* p, void* stream);

struct Buf {
    int dev, slot;
    void* stream;
    void* ptr;
    size_t bytes;
};

struct Shared {
    AllocFn alloc = nullptr;
    ReleaseFn release = nullptr;
    std::mutex mu;                 // guards orphans
    std::vector<Buf> orphans;
    std::atomic<long> live{0};     // buffers held by threads and orphans
};

inline Shared& shared() {
    static Shared* s = new Shared;  // never destroyed: thread tables may outlive static teardown
    return *s;
}

struct Table {
    std::vector<Buf> bufs;
    ~Table() {
        if (bufs.empty()) return;
        Shared& s = shared();
        std::lock_guard<std::mutex> lock(s.mu);
        s.orphans.insert(s.orphans.end(), bufs.begin(), bufs.end());
    }
};

inline Table& table() {
    thread_local Table t;
    return t;
}

inline void init(AllocFn alloc, ReleaseFn release) {
    Shared& s = shared();
    s.alloc = alloc;
    s.release = release;
}

// A buffer of at least `bytes` for this thread's work on (dev, stream, slot).
inline void* get(int dev, void* stream, int slot, size_t bytes, bool zeroed) {
    Shared& s = shared();
    Table& t = table();
    if (bytes == 0) bytes = 1;
    Buf* b = nullptr;
    for (auto& e : t.bufs)
        if (e.dev == dev && e.slot == slot && e.stream == stream) { b = &e; break; }
    if (!b) {
        // adopt the largest orphan of this key, if any
        std::lock_guard<std::mutex> lock(s.mu);
        size_t best = s.orphans.size();
        for (size_t i = 0; i < s.orphans.size(); i++) {
            const Buf& o = s.orphans[i];
            if (o.dev == dev && o.slot == slot && o.stream == stream &&
                (best == s.orphans.size() || o.bytes > s.orphans[best].bytes))
                best = i;
        }
        if (best < s.orphans.size()) {
            t.bufs.push_back(s.orphans[best]);
            s.orphans[best] = s.orphans.back();
            s.orphans.pop_back();
            b = &t.bufs.back();
        }
    }
    if (b && b->bytes >= bytes) return b->ptr;
    const size_t want = (bytes + (bytes >> 2) + 4095) & ~(size_t)4095;   // +25% headroom
    void* p = s.alloc(want, stream, zeroed);
    if (!p) return nullptr;
    if (b) {
        s.release(b->ptr, stream);
        b->ptr = p;
        b->bytes = want;
    } else {
        t.bufs.push_back(Buf{dev, slot, stream, p, want});
        s.live.fetch_add(1, std::memory_order_relaxed);
    }
    return p;
}

// Frees this thread's buffers and all orphans on `stream` (stream-ordered).
inline void release_stream(void* stream) {
    Shared& s = shared();
    Table& t = table();
    long n = 0;
    for (size_t i = 0; i < t.bufs.size();) {
        if (t.bufs[i].stream == stream) {
            s.release(t.bufs[i].ptr, stream);
            t.bufs[i] = t.bufs.back();
            t.bufs.pop_back();
            n++;
        } else {
            i++;
        }
    }
    {
        std::lock_guard<std::mutex> lock(s.mu);
        for (size_t i = 0; i < s.orphans.size();) {
            if (s.orphans[i].stream == stream) {
                s.release(s.orphans[i].ptr, stream);
                s.orphans[i] = s.orphans.back();
                s.orphans.pop_back();
                n++;
            } else {
                i++;
            }
        }
    }
    s.live.fetch_sub(n, std::memory_order_relaxed);
}

inline long live() { return shared().live.load(std::memory_order_relaxed); }

inline long orphan_count() {
    Shared& s = shared();
    std::lock_guard<std::mutex> lock(s.mu);
    return (long)s.orphans.size();
}

}  // namespace snx_ws

#endif  // SNX_WS_REGISTRY_H
