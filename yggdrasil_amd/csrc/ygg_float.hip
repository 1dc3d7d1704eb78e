// The float step of Yggdrasil (yggdrasil/inference.py:42-74): the inference model of a float checkpoint, in f32 for
// serving (the role of the Triton backend, yggdrasil/inference_triton.py) or f64 (the precision cpu/export.py
// calibrates in, cpu/export.py:101-153). One workgroup of 256 threads runs one stream through every layer of every
// token of a launch; the states of all layers stay in LDS.
//
// Per token x and layer l (expert r = x in the token layer, else the router's leaf):
//   route:   node = 1 .. 2^D - 1 (heap), right iff [router_embed[x]; rms(h_below)] . W[node] + b[node] > 0
//   update:  h = T_r[x];  h += U'_r (V' rms(h_below));  h += A_r h_old   (A_r block-diagonal)
//   readout: z = P_r h;   logits += Q z
// and rms(h) = h / sqrt(mean(h^2) + 1e-6) feeds the next layer.
// Work split: the router descends in rounds of up to 4 levels, 16 groups of 16 threads each forming one node's dot of
// the round's subtree (every load of a round issued at once, the input row held in registers for the layer); for the
// layer input wavefront q sums its quarter of the coordinates for row k = lane of V'; thread i owns coordinate i of
// the update (its table entry, U' column and A row loaded together); the readout takes 256 / R threads per row of P;
// thread c owns class c of the logits. The builds specialised on a shape issue a layer's constant loads (Q's column
// of each class, V''s share of each thread) at the layer's start, before its route, and the readout's P row with the
// update's record, so that a layer waits for the route's rounds and one record load only.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/ygg_hip.h"
#include "ygg_layout.h"

namespace ygg {
int set_error(int code, const char *msg);
}

namespace {

constexpr int kMaxN = 256, kMaxR = 64, kMaxR2 = 64, kMaxClasses = 256, kMaxF = 256, kMaxB = 16;
constexpr double kRmsEps = 1e-6;   // yggdrasil/config.py:8

// Device layouts: the arrays a thread reads a row of at each step of a dot are stored transposed from the checkpoint's,
// so that the lanes of a wavefront read consecutive addresses at every step.
template <typename T> struct FloatLayerDev {
    const T *table;          // token layer [V][n] (T_x[x]); routed [E][V][n]
    const T *A;              // [E][n/b][b (column j)][b (row i)] (each block transposed) or null
    const T *P;              // [E][R][n]
    const T *Q;              // [R][classes] (transposed)
    const T *emb;            // routed: [V][F]
    const T *W;              // routed: [nodes][F + n] (router_state) or [nodes][F]
    const T *bias;           // routed: [nodes]
    const T *Vd;             // [n][R2] (transposed) or null
    const T *Up;             // [E][R2][n] (each expert's matrix transposed) or null
};

template <typename T> struct FloatDevModel {
    int L, n, b, V, classes, D, R, R2, F, router_state;
    const T *output_bias;    // [classes]
    uint32_t *err;
    FloatLayerDev<T> layers[YGG_MAX_LAYERS];
};

constexpr int kFThreads = 256;

template <typename T> __device__ __forceinline__ T wave_sum(T v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <typename T> __device__ __forceinline__ T wave_max(T v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o));
    return v;
}

// the sum over aligned groups of G lanes (G a power of 2, at most 64), in every lane of the group
template <int G, typename T> __device__ __forceinline__ T group_sum(T v) {
    for (int o = G / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
template <typename T> __device__ __forceinline__ T group_sum_n(T v, int g) {
    for (int o = g / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
template <typename T> __device__ __forceinline__ T group_max_n(T v, int g) {
    for (int o = g / 2; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o));
    return v;
}

// atomic max of a non-negative double (its bit pattern orders as an unsigned integer)
__device__ __forceinline__ void atomic_max_nonneg(double *p, double v) {
    atomicMax((unsigned long long *)p, (unsigned long long)__double_as_longlong(v));
}

// the sum of v over the workgroup (red: 4 slots of LDS; two barriers)
template <typename T> __device__ __forceinline__ T block_sum(T v, T *red, int tid) {
    v = wave_sum(v);
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    const T s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

constexpr int kRouteGroup = 16;                           // threads per node of a router round
constexpr int kRouteElems = (kMaxF + kMaxN) / kRouteGroup; // router inputs per thread at most

// stats (calibration maxima, cpu/export.py:127-153), per layer: [|h|, |V' rms(h_below)|, |P_r h|, |h| per 16
// coordinates (n/16), |P_r h| per row (R)]
// NS, RS, R2S, BS: the state width, readout rank, layer-input rank and block size at compile time (the reference's
// trained shapes: every row length a constant), or 0 for the model's (any shape the loader takes)
// (one wavefront per SIMD: the unrolled row loads of a thread are its registers)
template <typename T, int NS = 0, int RS = 0, int R2S = 0, int BS = 0>
__global__ __launch_bounds__(kFThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void float_kernel(
    const FloatDevModel<T> m, const int32_t *__restrict__ tokens, int Tn, T *__restrict__ state,
    T *__restrict__ logits, int32_t *__restrict__ leaves, double *__restrict__ stats) {
    constexpr int MN = NS ? NS : kMaxN, MR = RS ? RS : kMaxR, MR2 = R2S ? R2S : kMaxR2, MB = BS ? BS : kMaxB;
    __shared__ T hs[YGG_MAX_LAYERS][kMaxN];   // states
    __shared__ T bl[kMaxN];                   // rms(h) of the layer below
    __shared__ T hn[kMaxN];                   // the new state of the current layer
    __shared__ T zl[kMaxR2];
    __shared__ T zs[kMaxR];
    __shared__ T zp[4][kMaxR2];               // the layer input's partial sums, per quarter of the coordinates
    __shared__ T red[4];
    __shared__ int dec[16];                   // a router round's decisions, by breadth-first node of its subtree
    __shared__ double gmax[YGG_MAX_LAYERS][kMaxN / 16];

    // PF (the specialised builds): a layer's loads issued early (see above); the general builds load at each use
    constexpr bool PF = NS != 0;
    constexpr int PE = RS ? (NS * RS + kFThreads - 1) / kFThreads : MN / 4;   // readout coordinates per thread
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int L = m.L, n = NS ? NS : m.n, b = BS ? BS : m.b, V = m.V, C = m.classes, R = RS ? RS : m.R,
              R2 = R2S ? R2S : m.R2, F = m.F;
    const int width = F + (m.router_state ? n : 0);
    // readout: TPR threads per row of P (a power of 2 of at most 64 lanes), its coordinates u, u + TPR, ...
    int Rp = 1;
    while (Rp < R) Rp <<= 1;
    const int TPR = kFThreads / Rp > 64 ? 64 : kFThreads / Rp;
    const int prow = tid / TPR, pu = tid % TPR;
    // layer input: wave q takes the quarter q of the coordinates, lane k row k of V'
    const int vrow = lane, vq = tid >> 6, vlen = n / 4;
    // router rounds: group g of kRouteGroup threads forms node g of the round's subtree
    const int rg = tid / kRouteGroup, rl = tid % kRouteGroup;

    T *st = state + (size_t)s * L * n;
    for (int l = 0; l < L; l++)
        for (int i = tid; i < n; i += kFThreads) hs[l][i] = st[(size_t)l * n + i];
    for (int l = 0; l < L; l++)
        for (int g = tid; g < n / 16; g += kFThreads) gmax[l][g] = 0.0;
    // per-thread maxima (calibration runs only): |h| (thread i's coordinate), |zl| (row vrow's reducer), |z| (row
    // prow's reducer)
    double smax[YGG_MAX_LAYERS], vmax[YGG_MAX_LAYERS], zmax[YGG_MAX_LAYERS];
    for (int l = 0; l < YGG_MAX_LAYERS; l++) smax[l] = vmax[l] = zmax[l] = 0.0;
    const int sstride = 3 + n / 16 + R;
    __syncthreads();

    const int32_t *tok = tokens + (size_t)s * Tn;
    for (int t = 0; t < Tn; t++) {
        const int x = __builtin_amdgcn_readfirstlane(tok[t]);
        if (x < 0 || x >= V) {
            if (tid == 0) atomicOr(m.err, 1u);
            break;
        }
        T lg = tid < C ? m.output_bias[tid] : T(0);
        for (int l = 0; l < L; l++) {
            const FloatLayerDev<T> &y = m.layers[l];
            int r = x;
            // the layer's constants: class c's column of Q^T (thread c) and this thread's share of V' (wave q's quarter
            // of the coordinates of row k = lane)
            T qw[MR], vv[MN / 4];
            auto load_q = [&]() {
                if (tid < C) {
                    const T *q = y.Q + tid;
#pragma unroll
                    for (int j = 0; j < MR; j++) qw[j] = j < R ? q[(size_t)j * C] : T(0);
                }
            };
            const bool vlive = l > 0 && y.Vd != nullptr && vrow < R2;
            auto load_v = [&]() {
                if (vlive) {
                    const T *vc = y.Vd + (size_t)(vq * vlen) * R2 + vrow;
#pragma unroll
                    for (int i = 0; i < MN / 4; i++) vv[i] = i < vlen ? vc[(size_t)i * R2] : T(0);
                }
            };
            if constexpr (PF) {
                load_q();
                load_v();
            }
            if (l > 0) {
                // router descent over f = [router_embed[x]; rms(h_below)], in rounds of up to 4 levels
                T f[kRouteElems];
                const T *e = y.emb + (size_t)x * F;
#pragma unroll
                for (int k = 0; k < kRouteElems; k++) {
                    const int i = rl + kRouteGroup * k;
                    f[k] = i < F ? e[i] : (i < width ? bl[i - F] : T(0));
                }
                int root = 0;
                for (int d0 = 0; d0 < m.D; d0 += 4) {
                    const int h = m.D - d0 < 4 ? m.D - d0 : 4;
                    const int nn = (1 << h) - 1;
                    // node rg of the subtree: depth k = floor(log2(rg + 1)), path p = rg + 1 - 2^k
                    const int kdep = 31 - __builtin_clz(rg + 1), path = rg + 1 - (1 << kdep);
                    const int node = ((root + 1) << kdep) - 1 + path;
                    T p = T(0);
                    if (rg < nn) {
                        const T *w = y.W + (size_t)node * width;
                        T wl[kRouteElems];
#pragma unroll
                        for (int k = 0; k < kRouteElems; k++) {
                            const int i = rl + kRouteGroup * k;
                            wl[k] = i < width ? w[i] : T(0);
                        }
#pragma unroll
                        for (int k = 0; k < kRouteElems; k++) p += f[k] * wl[k];
                    }
                    p = group_sum<kRouteGroup>(p);
                    if (rg < nn && rl == 0) dec[rg] = (p + y.bias[node]) > T(0) ? 1 : 0;
                    __syncthreads();
                    int q = 0;
                    for (int k = 0; k < h; k++) q = 2 * q + dec[(1 << k) - 1 + q];
                    root = ((root + 1) << h) - 1 + q;
                    __syncthreads();
                }
                r = root - ((1 << m.D) - 1);
                // the layer input zl = V' rms(h_below): each wave's partial sum for row k = lane over its quarter of
                // the coordinates, the four partials then added in quarter order
                if (y.Vd) {
                    if constexpr (!PF) load_v();
                    if (vlive) {
                        T a = T(0);
#pragma unroll
                        for (int i = 0; i < MN / 4; i++)
                            if (i < vlen) a += vv[i] * bl[vq * vlen + i];
                        zp[vq][vrow] = a;
                    }
                    __syncthreads();
                    if (tid < R2) {
                        const T z = ((zp[0][tid] + zp[1][tid]) + zp[2][tid]) + zp[3][tid];
                        zl[tid] = z;
                        if (stats) vmax[l] = fmax(vmax[l], (double)fabs(z));
                    }
                    __syncthreads();
                }
            }
            // expert r's P row share for the readout: TPR threads per row, coordinates pu, pu + TPR, ...
            T pw[PE];
            auto load_p = [&]() {
                if (prow < R) {
                    const T *pr = y.P + ((size_t)r * R + prow) * n;
#pragma unroll
                    for (int e = 0; e < PE; e++) pw[e] = pu + TPR * e < n ? pr[pu + TPR * e] : T(0);
                }
            };
            // h = T_r[x] + U'_r zl + A_r h_old, thread i for coordinate i
            T hv = T(0);
            if (tid < n) {
                // (the table entry, U' column and A row of coordinate i loaded together; sums in index order)
                const int i = tid;
                const T *trow = l == 0 ? y.table + (size_t)x * n : y.table + ((size_t)r * V + x) * n;
                const bool up = l > 0 && y.Up != nullptr, ta = y.A != nullptr;
                const int g = i / b, ii = i % b;
                const T *u = up ? y.Up + (size_t)r * R2 * n + i : nullptr;                    // column i
                const T *acol = ta ? y.A + ((size_t)r * (n / b) + g) * b * b + ii : nullptr;  // row ii of block g
                T uw[MR2], aw[MB];
#pragma unroll
                for (int k = 0; k < MR2; k++) uw[k] = (up && k < R2) ? u[(size_t)k * n] : T(0);
#pragma unroll
                for (int j = 0; j < MB; j++) aw[j] = (ta && j < b) ? acol[j * b] : T(0);
                T h = trow[i];
                if constexpr (PF) load_p();
                if (up) {
                    T a = T(0);
#pragma unroll
                    for (int k = 0; k < MR2; k++)
                        if (k < R2) a += uw[k] * zl[k];
                    h = h + a;
                }
                if (ta) {
                    T a = T(0);
#pragma unroll
                    for (int j = 0; j < MB; j++)
                        if (j < b) a += aw[j] * hs[l][g * b + j];
                    h = h + a;
                }
                hv = h;
                if (stats) smax[l] = fmax(smax[l], (double)fabs(h));
            } else if constexpr (PF) {
                load_p();
            }
            // (every thread has read hs[l] before it is overwritten below)
            const T ss = block_sum(tid < n ? hv * hv : T(0), red, tid);
            if (tid < n) {
                hn[tid] = hv;
                hs[l][tid] = hv;
            }
            if (stats && tid < n) {
                // |h| per 16 coordinates: 16 consecutive threads
                const double a = group_max_n((double)fabs(hv), 16);
                if ((tid & 15) == 0) gmax[l][tid >> 4] = fmax(gmax[l][tid >> 4], a);
            }
            const T rinv = T(1) / sqrt(ss / T(n) + T(kRmsEps));
            if (tid < n) bl[tid] = hv * rinv;
            __syncthreads();
            // z = P_r h (every load issued at once)
            if constexpr (!PF) load_p();
            if (prow < R) {
                T a = T(0);
#pragma unroll
                for (int e = 0; e < PE; e++)
                    if (pu + TPR * e < n) a += pw[e] * hn[pu + TPR * e];
                a = group_sum_n(a, TPR);
                if (pu == 0) {
                    zs[prow] = a;
                    if (stats) zmax[l] = fmax(zmax[l], (double)fabs(a));   // row prow's reducer holds its maximum
                }
            }
            __syncthreads();
            // logits += Q z, thread c for class c
            if constexpr (!PF) load_q();
            if (tid < C) {
                T a = T(0);
#pragma unroll
                for (int j = 0; j < MR; j++)
                    if (j < R) a += qw[j] * zs[j];
                lg = lg + a;
            }
            if (leaves && tid == 0) leaves[((size_t)s * Tn + t) * L + l] = r;
            __syncthreads();
        }
        if (logits && tid < C) logits[((size_t)s * Tn + t) * C + tid] = lg;
    }
    __syncthreads();
    for (int l = 0; l < L; l++)
        for (int i = tid; i < n; i += kFThreads) st[(size_t)l * n + i] = hs[l][i];
    if (stats) {
        for (int l = 0; l < L; l++) {
            const double a = wave_max(smax[l]), v = wave_max(vmax[l]), z = wave_max(zmax[l]);
            if (lane == 0) {
                atomic_max_nonneg(&stats[(size_t)l * sstride + 0], a);
                atomic_max_nonneg(&stats[(size_t)l * sstride + 1], v);
                atomic_max_nonneg(&stats[(size_t)l * sstride + 2], z);
            }
            for (int g = tid; g < n / 16; g += kFThreads)
                atomic_max_nonneg(&stats[(size_t)l * sstride + 3 + g], gmax[l][g]);
            if (prow < R && pu == 0) atomic_max_nonneg(&stats[(size_t)l * sstride + 3 + n / 16 + prow], zmax[l]);
        }
    }
}

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return ygg::set_error(code, buf);
}

#define HIP_TRY(expr)                                                                                  \
    do {                                                                                               \
        hipError_t e_ = (expr);                                                                        \
        if (e_ != hipSuccess) return fail(YGG_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_));     \
    } while (0)

struct DeviceGuard {
    int prev = -1;
    hipError_t set(int dev) {
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) { prev = -1; return e; }
        return hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

}  // namespace

struct ygg_fmodel {
    int device = 0, precision = 32;
    void *arena = nullptr;
    size_t arena_bytes = 0;
    FloatDevModel<float> m32{};
    FloatDevModel<double> m64{};
};

namespace {

template <typename T> int upload(const ygg_float_desc *d, int device, ygg_fmodel *fm, FloatDevModel<T> &m) {
    const int L = d->n_layers, n = d->d_state, b = d->block_size, V = d->vocab, C = d->classes, D = d->router_depth,
              R = d->readout_rank, R2 = d->layer_input_rank, F = d->router_token_dim;
    const int64_t E = (int64_t)1 << D, nodes = E - 1, width = F + (d->router_state ? n : 0);
    // a part is `outer` matrices of rows x cols, stored as given (rows = 0) or each transposed
    struct Part { const double *src; int64_t count; size_t off; int64_t outer, rows, cols; };
    std::vector<Part> parts;
    size_t total = 256;   // the error word first
    auto add = [&](const double *src, int64_t count, int64_t rows = 0, int64_t cols = 0) -> int {
        if (!src || count <= 0) return -1;
        parts.push_back({src, count, total, rows ? count / (rows * cols) : 0, rows, cols});
        total += ((size_t)count * sizeof(T) + 255) / 256 * 256;
        return (int)parts.size() - 1;
    };
    const int ob = add(d->output_bias, C);
    if (ob < 0) return fail(YGG_ERR_ARG, "float model: output_bias is NULL");
    struct Idx { int table, A, P, Q, emb, W, bias, Vd, Up; };
    std::vector<Idx> idx(L);
    for (int l = 0; l < L; l++) {
        const ygg_float_layer &y = d->layers[l];
        const int64_t El = l == 0 ? V : E;
        Idx &k = idx[l];
        k.table = add(y.table, l == 0 ? (int64_t)V * n : El * V * n);
        k.A = add(y.transition, El * n * b, b, b);
        k.P = add(y.readout, El * R * n);
        k.Q = add(y.unembed, (int64_t)C * R, C, R);
        k.emb = l ? add(y.router_embed, (int64_t)V * F) : -1;
        k.W = l ? add(y.router_weight, nodes * width) : -1;
        k.bias = l ? add(y.router_bias, nodes) : -1;
        k.Vd = (l && R2) ? add(y.layer_input_down, (int64_t)R2 * n, R2, n) : -1;
        k.Up = (l && R2) ? add(y.layer_input_proj, El * n * R2, n, R2) : -1;
        if (k.table < 0 || k.P < 0 || k.Q < 0 || (l && (k.emb < 0 || k.W < 0 || k.bias < 0)) ||
            (l && R2 && (k.Vd < 0 || k.Up < 0)))
            return fail(YGG_ERR_ARG, "float model: layer %d lacks an array", l);
    }
    // the description is checked before any device is touched
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(YGG_ERR_DEVICE, "no HIP device");
    if (device < 0 || device >= ndev) return fail(YGG_ERR_ARG, "device %d out of range", device);
    std::vector<uint8_t> host;
    try {
        host.assign(total, 0);
    } catch (const std::bad_alloc &) {
        return fail(YGG_ERR_NOMEM, "float model: %zu bytes of host staging", total);
    }
    for (const Part &p : parts) {
        T *dst = (T *)(host.data() + p.off);
        if (!p.rows) {
            for (int64_t i = 0; i < p.count; i++) dst[i] = (T)p.src[i];
            continue;
        }
        const int64_t mat = p.rows * p.cols;
        for (int64_t o = 0; o < p.outer; o++)
            for (int64_t r = 0; r < p.rows; r++)
                for (int64_t c = 0; c < p.cols; c++) dst[o * mat + c * p.rows + r] = (T)p.src[o * mat + r * p.cols + c];
    }
    DeviceGuard g;
    HIP_TRY(g.set(device));
    void *arena = nullptr;
    HIP_TRY(hipMalloc(&arena, total));
    hipError_t e = hipMemcpy(arena, host.data(), total, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(arena);
        return fail(YGG_ERR_DEVICE, "upload failed: %s", hipGetErrorString(e));
    }
    uint8_t *A = (uint8_t *)arena;
    auto at = [&](int i) -> const T * { return i < 0 ? nullptr : (const T *)(A + parts[i].off); };
    m.L = L; m.n = n; m.b = b; m.V = V; m.classes = C; m.D = D; m.R = R; m.R2 = R2; m.F = F;
    m.router_state = d->router_state;
    m.output_bias = at(ob);
    m.err = (uint32_t *)arena;
    for (int l = 0; l < L; l++) {
        const Idx &k = idx[l];
        m.layers[l] = FloatLayerDev<T>{at(k.table), at(k.A), at(k.P), at(k.Q), at(k.emb), at(k.W), at(k.bias),
                                       at(k.Vd), at(k.Up)};
    }
    fm->arena = arena;
    fm->arena_bytes = total;
    return YGG_OK;
}

}  // namespace

extern "C" {

int ygg_float_load(const ygg_float_desc *d, int precision, int device, ygg_fmodel **out) {
    if (!out) return fail(YGG_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (!d) return fail(YGG_ERR_ARG, "desc is NULL");
    if (precision != 32 && precision != 64) return fail(YGG_ERR_ARG, "precision %d: 32 or 64", precision);
    const int L = d->n_layers, n = d->d_state, b = d->block_size;
    if (L < 1 || L > YGG_MAX_LAYERS || n < 16 || n > kMaxN || n % 16 || b < 1 || b > kMaxB || n % b || d->vocab < 1 ||
        d->classes < 1 || d->classes > kMaxClasses || d->readout_rank < 1 || d->readout_rank > kMaxR ||
        d->layer_input_rank < 0 || d->layer_input_rank > kMaxR2 || (L > 1 && (d->router_depth < 1 ||
        d->router_depth > 20 || d->router_token_dim < 0 || d->router_token_dim > kMaxF)))
        return fail(YGG_ERR_LIMITS, "float model: unsupported shape (L %d, n %d, b %d, classes %d, R %d, R2 %d, D %d)",
                    L, n, b, d->classes, d->readout_rank, d->layer_input_rank, d->router_depth);
    ygg_fmodel *fm = new ygg_fmodel();
    fm->device = device;
    fm->precision = precision;
    const int rc = precision == 32 ? upload<float>(d, device, fm, fm->m32) : upload<double>(d, device, fm, fm->m64);
    if (rc != YGG_OK) {
        delete fm;
        return rc;
    }
    *out = fm;
    return YGG_OK;
}

int ygg_float_run(const ygg_fmodel *m, const int32_t *d_tokens, int B, int T, void *d_state, void *d_logits,
                  int32_t *d_leaves, double *d_stats, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0 || T < 0) return fail(YGG_ERR_ARG, "negative B (%d) or T (%d)", B, T);
    if (B == 0) return YGG_OK;
    if (!d_state || (T > 0 && !d_tokens)) return fail(YGG_ERR_ARG, "tokens or state is NULL");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    if (m->precision == 32) {
        // the reference's trained shapes (configs/*/{small,medium,large}.yaml: block 16) have builds of their own
        const FloatDevModel<float> &fm = m->m32;
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(B), dim3(kFThreads), 0, (hipStream_t)stream, fm, d_tokens, T,
                               (float *)d_state, (float *)d_logits, d_leaves, d_stats);
        };
        if (fm.b == 16 && fm.n == 64 && fm.R == 8 && fm.R2 == 16) go(float_kernel<float, 64, 8, 16, 16>);
        else if (fm.b == 16 && fm.n == 128 && fm.R == 16 && fm.R2 == 32) go(float_kernel<float, 128, 16, 32, 16>);
        else if (fm.b == 16 && fm.n == 256 && fm.R == 32 && fm.R2 == 64) go(float_kernel<float, 256, 32, 64, 16>);
        else go(float_kernel<float>);
    } else
        hipLaunchKernelGGL(float_kernel<double>, dim3(B), dim3(kFThreads), 0, (hipStream_t)stream, m->m64, d_tokens, T,
                           (double *)d_state, (double *)d_logits, d_leaves, d_stats);
    HIP_TRY(hipGetLastError());
    return YGG_OK;
}

int ygg_float_take_errors(const ygg_fmodel *m, void *stream, uint32_t *errors) {
    if (!m || !errors) return fail(YGG_ERR_ARG, "NULL argument");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    uint32_t v = 0;
    HIP_TRY(hipMemcpy(&v, m->arena, 4, hipMemcpyDeviceToHost));
    if (v) {
        const uint32_t zero = 0;
        HIP_TRY(hipMemcpy(m->arena, &zero, 4, hipMemcpyHostToDevice));
    }
    *errors = v;
    return YGG_OK;
}

void ygg_float_free(ygg_fmodel *m) {
    if (!m) return;
    DeviceGuard g;
    if (g.set(m->device) == hipSuccess) (void)hipFree(m->arena);
    delete m;
}

}  // extern "C"
