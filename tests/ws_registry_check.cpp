// CPU check of the workspace registry (sneppx-alg_amd/csrc/ws_registry.h)
// with a counting malloc allocator in place of the device pool.  Built and
// run by tests/test_ws_registry.py; exit status 0 when every check holds.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <set>
#include <thread>
#include <vector>

#include "ws_registry.h"

static std::atomic<long> g_outstanding{0};
static std::atomic<long> g_allocs{0};

static void* fake_alloc(size_t bytes, void*, bool zeroed) {
    g_allocs++;
    g_outstanding++;
    return zeroed ? calloc(1, bytes) : malloc(bytes);
}

static void fake_release(void* p, void*) {
    g_outstanding--;
    free(p);
}

#define CHECK(c)                                                          \
    do {                                                                  \
        if (!(c)) {                                                       \
            fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
            return 1;                                                     \
        }                                                                 \
    } while (0)

int main() {
    snx_ws::init(fake_alloc, fake_release);
    void* const S1 = (void*)0x1000;
    void* const S2 = (void*)0x2000;
    CHECK(snx_ws::live() == 0);

    // one thread: reuse, growth (old buffer released), separate slots/streams
    void* a = snx_ws::get(0, S1, 0, 1000, false);
    CHECK(a && snx_ws::get(0, S1, 0, 800, false) == a);
    void* b = snx_ws::get(0, S1, 0, 100000, false);
    CHECK(b && b != a && snx_ws::live() == 1 && g_outstanding == 1);
    void* c = snx_ws::get(0, S1, 1, 64, true);
    void* d = snx_ws::get(0, S2, 0, 64, false);
    CHECK(c && d && c != b && d != b && snx_ws::live() == 3);

    // many short-lived threads, at most 4 alive at once, each using 2
    // streams x 3 slots with sizes that grow: the buffers they leave are
    // adopted by later threads, so the count stays at (threads alive at
    // once) x streams x slots, not (threads ever) x streams x slots
    const long before = snx_ws::live();
    std::mutex mu;
    bool distinct = true;
    for (int wave = 0; wave < 50; wave++) {
        std::set<void*> seen;
        std::vector<std::thread> ts;
        std::atomic<int> arrived{0};
        for (int t = 0; t < 4; t++)
            ts.emplace_back([&, wave, t] {
                std::vector<void*> mine;
                for (void* s : {S1, S2})
                    for (int slot = 0; slot < 3; slot++) {
                        void* p = snx_ws::get(0, s, slot, 256 + 64 * (size_t)(wave % 7) + t, slot == 2);
                        if (p) mine.push_back(p);
                    }
                {
                    std::lock_guard<std::mutex> lock(mu);
                    for (void* p : mine)
                        if (!seen.insert(p).second) distinct = false;   // two live threads share a buffer
                }
                // stay alive until all four hold their buffers, so none of
                // them can have been handed on yet
                arrived++;
                while (arrived.load() < 4) std::this_thread::yield();
            });
        for (auto& th : ts) th.join();
    }
    CHECK(distinct);
    const long grown = snx_ws::live() - before;
    CHECK(grown <= 4 * 2 * 3);
    CHECK(snx_ws::orphan_count() == grown);
    CHECK(g_outstanding == snx_ws::live());

    // releasing the two streams frees this thread's buffers and the orphans
    snx_ws::release_stream(S1);
    snx_ws::release_stream(S2);
    CHECK(snx_ws::live() == 0 && snx_ws::orphan_count() == 0 && g_outstanding == 0);
    printf("ok: %ld allocations, %ld workspaces at most after 200 threads\n", (long)g_allocs, grown);
    return 0;
}
