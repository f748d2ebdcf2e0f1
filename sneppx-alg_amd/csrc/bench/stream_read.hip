// stream_read.hip - a plain streaming read for bench.py's intercept fit (not
// part of the product library): the M = 1 W4A16 GEMV's memory access shape
// with no arithmetic.  512 threads per workgroup, every thread four 16-byte
// nontemporal loads, each wave instruction 1 KB contiguous, all in flight at
// once; the loaded words are XOR-folded and stored only if the fold equals a
// value the caller never passes, so the loads cannot be removed.  Launched
// back to back over rotating buffers it gives what a launch of that shape
// costs beyond its bytes.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {
constexpr int kThreads = 512, kLoads = 4;
constexpr int kNontemporal = 2;   // buffer cache policy: nt

__global__ void __launch_bounds__(kThreads) k_stream_read(const uint32_t* __restrict__ src, uint32_t n16,
                                                          uint32_t magic, uint32_t* __restrict__ sink) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), (short)0,
                                                                       (int)(n16 * 16u), 0x00020000);
    const uint32_t base = blockIdx.x * (kThreads * kLoads) + (threadIdx.x & ~63u) * kLoads + (threadIdx.x & 63u);
    uint32_t acc = 0u;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; i++) {
        const uint32_t c = base + 64u * i;   // the wave's i-th 1 KB piece
        v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, c < n16 ? c * 16u : 0x80000000u,
                                                                               0, kNontemporal));
    }
#pragma unroll
    for (int i = 0; i < kLoads; i++) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    if (acc == magic) sink[0] = acc;
}
}  // namespace

// Reads `bytes` (a multiple of 16, below 2 GiB) of `src` on `stream`.
extern "C" int snxb_stream_read(const void* src, size_t bytes, void* sink, void* stream) {
    if (bytes % 16 || bytes >= (1ull << 31)) return -1;
    const uint32_t n16 = (uint32_t)(bytes / 16);
    const uint32_t per = kThreads * kLoads;
    k_stream_read<<<(n16 + per - 1) / per, kThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const uint32_t*>(src), n16, 0xA5C3E1F7u, static_cast<uint32_t*>(sink));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
