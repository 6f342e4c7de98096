// qr_floor.hip -- a plain streaming read, the measurement helper behind bench.py's
// stream_floor_us (built as its own library, libqr_floor.so; not part of the attention
// library or its C ABI).
//
// Every byte of a buffer is read once with non-temporal 16-byte loads and nothing is
// computed: one contiguous chunk per 256-thread workgroup, eight loads in flight per
// thread.  Its time for the byte count of a workload is what HBM delivers on the same GPU,
// in the same process, to a kernel that does nothing else -- the practical floor of an
// HBM-bound call of that many bytes.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) floor_read_kernel(const u32x4* __restrict__ p, size_t n, unsigned* sink) {
    unsigned acc = 0;
    const size_t per = (n + gridDim.x - 1) / gridDim.x;
    const size_t b0 = static_cast<size_t>(blockIdx.x) * per;
    const size_t b1 = b0 + per < n ? b0 + per : n;
    for (size_t i = b0 + threadIdx.x; i < b1; i += 256 * 8) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const size_t j = i + 256 * u;
            v[u] = j < b1 ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    // keeps the loads alive; taken only when the XOR of a chunk happens to hit the constant
    if (acc == 0x9E3779B9u) sink[blockIdx.x & 63] = acc;
}

}  // namespace

// `reps` reads launched back to back on `stream`, read r covering set r % sets of the
// buffer (sets of set_bytes each, contiguous from buf); sink holds 64 unsigned ints.
// Returns 0, 1 for invalid arguments, 2 for a launch error.
extern "C" int qr_floor_read(const void* buf, size_t set_bytes, int sets, int reps, unsigned* sink, int blocks,
                             void* stream) {
    if (!buf || !sink || set_bytes < 16 || set_bytes % 16 || sets < 1 || reps < 1 || blocks < 1 || blocks > 65535 ||
        reinterpret_cast<uintptr_t>(buf) % 16)
        return 1;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int r = 0; r < reps; ++r) {
        const char* set = static_cast<const char*>(buf) + static_cast<size_t>(r % sets) * set_bytes;
        hipLaunchKernelGGL(floor_read_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const u32x4*>(set),
                           set_bytes / 16, sink);
        if (hipGetLastError() != hipSuccess) return 2;
    }
    return 0;
}
