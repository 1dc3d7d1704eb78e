// Measurement probe (libygg_probe.so, used by bench.py --probe only): the memory pattern of the batched step without
// its arithmetic, to measure what the memory system delivers for it on this GPU.
//
// Each wavefront runs `chains` independent chains of `steps` gathers; a gather reads one record of rec_bytes (a
// multiple of 1024) at a pseudo-random record index of a buffer, as 16-byte loads, one contiguous KiB per load
// instruction (the step kernel's record loads). With dependent != 0 the next index of a chain depends on the bytes
// just read, so a chain has one gather in flight at a time, as a stream of the step kernel has; otherwise the indices
// come from a counter and the loads of successive gathers may overlap.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__device__ __forceinline__ uint64_t probe_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <int CH>
__global__ __launch_bounds__(256) void gather_probe(const uint4 *__restrict__ buf, uint64_t nrec, int rec16,
                                                    int steps, int dependent, unsigned *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const uint64_t w = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    uint64_t idx[CH];
    unsigned acc[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        idx[c] = probe_mix(w * CH + c);
        acc[c] = 0u;
    }
    for (int t = 0; t < steps; t++) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const uint4 *p = buf + (idx[c] % nrec) * (uint64_t)rec16;
            unsigned a = 0u;
            for (int k = 0; k < rec16; k += 64) {
                const uint4 v = p[k + lane];
                a ^= v.x + v.y + v.z + v.w;
            }
            acc[c] += a;
            const unsigned d = dependent ? (unsigned)__builtin_amdgcn_readfirstlane((int)(a & 1u)) : 0u;
            idx[c] = probe_mix(idx[c] + (uint64_t)t + d);
        }
    }
    unsigned r = 0u;
#pragma unroll
    for (int c = 0; c < CH; c++) r += acc[c];
    out[w * 64 + lane] = r;
}

}  // namespace

// Gathers of rec_bytes records from the bytes at buf by `waves` wavefronts (a multiple of 4), `chains` (1, 2 or 4)
// chains each, `steps` gathers per chain; out: waves * 64 words. Returns a hipError_t.
extern "C" int ygg_probe_gather(const void *buf, uint64_t bytes, int rec_bytes, int waves, int chains, int steps,
                                int dependent, unsigned *out, hipStream_t stream) {
    if (!buf || !out || rec_bytes <= 0 || rec_bytes % 1024 || waves <= 0 || waves % 4 || steps < 0 ||
        bytes < (uint64_t)rec_bytes)
        return (int)hipErrorInvalidValue;
    const uint64_t nrec = bytes / (uint64_t)rec_bytes;
    const dim3 grid(waves / 4), block(256);
    const int rec16 = rec_bytes / 16;
    const uint4 *b = (const uint4 *)buf;
    if (chains == 1)
        hipLaunchKernelGGL(gather_probe<1>, grid, block, 0, stream, b, nrec, rec16, steps, dependent, out);
    else if (chains == 2)
        hipLaunchKernelGGL(gather_probe<2>, grid, block, 0, stream, b, nrec, rec16, steps, dependent, out);
    else if (chains == 4)
        hipLaunchKernelGGL(gather_probe<4>, grid, block, 0, stream, b, nrec, rec16, steps, dependent, out);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}
