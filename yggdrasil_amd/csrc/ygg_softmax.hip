// The f32 softmax of the reference's `time` mode (cpu/ygg.cpp:44-72, called once per token at 545-553): for each row
// of V <= 256 logits, probabilities p_i = e_i * (1 / tot) and the row's log-sum-exp mx + log(tot), where
//   mx  = max_i lg_i
//   e_i = 2^n * P(f), t = clamp(lg_i - mx, -87, 88) * f32(log2 e), n = t rounded to nearest even, f = t - n, P the
//         degree-6 polynomial of the reference in Horner form with fused multiply-adds (cpu/ygg.cpp:48-55)
//   tot = the 16 sums s_j = sum over k (ascending) of e_(16 k + j), joined pairwise as s_j + s_(j+8), then 4 apart,
//         2 apart, 1 apart: the 16-lane accumulator and halving reduction of the reference's vector code
// so the probabilities equal the reference's to the bit (division correctly rounded, fma fused, exact scaling); the
// log-sum-exp uses the device's logf, within an ulp of the host's.
//
// One wavefront per row (lane l holds classes 4 l .. 4 l + 3), 4 per workgroup, rows strided over the grid, the next
// row's logits loaded while a row is reduced. The probabilities may overwrite the logits in place: a lane reads its
// classes of a row before it writes them, and the next row it has loaded ahead is not written by anyone before it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ygg_launch.h"

namespace ygg {

__device__ __forceinline__ float vexp_ref(float x) {
    x = fminf(fmaxf(x, -87.f), 88.f);
    const float t = x * 1.4426950408889634f;
    const float n = __builtin_rintf(t);
    const float f = t - n;
    float p = 1.5353362e-4f;
    p = __builtin_fmaf(p, f, 1.3398874e-3f);
    p = __builtin_fmaf(p, f, 9.6181291e-3f);
    p = __builtin_fmaf(p, f, 5.5504109e-2f);
    p = __builtin_fmaf(p, f, 2.4022651e-1f);
    p = __builtin_fmaf(p, f, 6.9314718e-1f);
    p = __builtin_fmaf(p, f, 1.0f);
    return __builtin_amdgcn_ldexpf(p, (int)n);
}

// the 4 logits of lane `lane` in row r (padding -inf): one 16-byte load when V is a multiple of 4
template <bool VEC>
__device__ __forceinline__ void load_row(float (&v)[4], const float *lg, int64_t r, int V, int lane) {
    if constexpr (VEC) {
        const float4 q = *(const float4 *)(lg + r * V + 4 * (4 * lane < V ? lane : 0));
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
        if (4 * lane >= V) v[0] = v[1] = v[2] = v[3] = -INFINITY;
    } else {
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = 4 * lane + u < V ? lg[r * V + 4 * lane + u] : -INFINITY;
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void softmax_kernel(const float *lg, int64_t rows, int V, float *pr, float *lse) {
    __shared__ float es[4][256];
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    float *e = es[wv];
    const int64_t stride = (int64_t)gridDim.x * 4;
    int64_t r = (int64_t)blockIdx.x * 4 + wv;
    if (r >= rows) return;
    float v[4];
    load_row<VEC>(v, lg, r, V, lane);
    for (; r < rows; r += stride) {
        // the next row's logits are loaded while this row is reduced (its address clamped to this row at the end)
        float nv[4];
        load_row<VEC>(nv, lg, r + stride < rows ? r + stride : r, V, lane);
        float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float ev[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            ev[u] = 4 * lane + u < V ? vexp_ref(v[u] - mx) : 0.0f;
            e[4 * lane + u] = ev[u];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lane j < 16: accumulator j, its terms in class order
        float s = 0.0f;
        if (lane < 16)
            for (int i = lane; i < V; i += 16) s = s + e[i];
        s = s + __shfl_down(s, 8);
        s = s + __shfl_down(s, 4);
        s = s + __shfl_down(s, 2);
        s = s + __shfl_down(s, 1);
        const float tot = __shfl(s, 0);
        const float inv = 1.0f / tot;
        float *out = pr + r * V;
        if constexpr (VEC) {
            if (4 * lane < V)
                *(float4 *)(out + 4 * lane) = make_float4(ev[0] * inv, ev[1] * inv, ev[2] * inv, ev[3] * inv);
        } else {
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (4 * lane + u < V) out[4 * lane + u] = ev[u] * inv;
        }
        if (lse && lane == 0) lse[r] = mx + logf(tot);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = nv[u];
    }
}

hipError_t launch_softmax(const float *logits, int64_t rows, int V, float *probs, float *lse, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    int64_t g = (rows + 3) / 4;
    if (g > 16384) g = 16384;
    // 16-byte loads and stores when every row starts 16-byte aligned
    const bool vec = V % 4 == 0 && ((uintptr_t)logits | (uintptr_t)probs) % 16 == 0;
    if (vec)
        hipLaunchKernelGGL(softmax_kernel<true>, dim3((unsigned)g), dim3(256), 0, stream, logits, rows, V, probs, lse);
    else
        hipLaunchKernelGGL(softmax_kernel<false>, dim3((unsigned)g), dim3(256), 0, stream, logits, rows, V, probs, lse);
    return hipGetLastError();
}

}  // namespace ygg
