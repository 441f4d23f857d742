// Read-only streaming probe for the measurement harness: the HBM read rate a plain streaming
// kernel reaches on this GPU, reported beside the GEMV's as a reference rate.  Block b reads its own
// contiguous share of the buffer front to back; each thread keeps 16 loads of 16 bytes in flight
// before it uses any of them (the block's loads in flight cover 128 KB of consecutive bytes), and
// XORs them; block b stores its XOR in out[b] (so the reads cannot be dropped, and a test can
// check them).
#include "tfp8_common.h"

namespace tfp8 {

namespace {

constexpr int RP_THREADS = 512, RP_DEPTH = 16;

__global__ __launch_bounds__(RP_THREADS) void read_probe_kernel(const uint4* __restrict__ p, int64_t n16,
                                                                uint32_t* __restrict__ out) {
    __shared__ uint32_t red[RP_THREADS / 64];
    const int64_t share = ((n16 + gridDim.x - 1) / gridDim.x + RP_THREADS - 1) / RP_THREADS * RP_THREADS;
    const int64_t beg = (int64_t)blockIdx.x * share, end = min(n16, beg + share);
    uint32_t acc = 0;
    for (int64_t base = beg + threadIdx.x; base < end; base += (int64_t)RP_THREADS * RP_DEPTH) {
        uint4 v[RP_DEPTH];
#pragma unroll
        for (int u = 0; u < RP_DEPTH; ++u) {
            const int64_t i = base + (int64_t)u * RP_THREADS;
            v[u] = i < end ? p[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < RP_DEPTH; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < RP_THREADS / 64; ++w) t ^= red[w];
        out[blockIdx.x] = t;
    }
}

}  // namespace

}  // namespace tfp8

extern "C" int tfp8_read_probe(const void* p, size_t bytes, uint32_t* out, int blocks, void* stream) {
    using namespace tfp8;
    clear_error();
    if (!p || !out || bytes % 16 || (uintptr_t)p % 16 || blocks <= 0 || blocks > 65536)
        return fail(TFP8_ERR_ARG, "tfp8_read_probe: 16-byte aligned buffer of a multiple of 16 bytes and 1..65536 blocks expected");
    if (bytes == 0) return 0;
    read_probe_kernel<<<blocks, RP_THREADS, 0, (hipStream_t)stream>>>((const uint4*)p, (int64_t)(bytes / 16), out);
    return check_launch("tfp8_read_probe");
}
