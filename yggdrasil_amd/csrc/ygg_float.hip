// The float step of Yggdrasil (yggdrasil/inference.py:42-74): the inference model of a float checkpoint, in f32 for
// serving (the role of the Triton backend, yggdrasil/inference_triton.py) or f64 (the precision cpu/export.py
// calibrates in, cpu/export.py:101-153). One 64-lane wavefront runs one stream through every layer of every token of
// a launch; the states of all layers stay in LDS.
//
// Per token x and layer l (expert r = x in the token layer, else the router's leaf):
//   route:   node = 1 .. 2^D - 1 (heap), right iff [router_embed[x]; rms(h_below)] . W[node] + b[node] > 0
//   update:  h = T_r[x];  h += U'_r (V' rms(h_below));  h += A_r h_old   (A_r block-diagonal)
//   readout: z = P_r h;   logits += Q z
// and rms(h) = h / sqrt(mean(h^2) + 1e-6) feeds the next layer. Lane i owns coordinates i, i + 64, ...
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

constexpr int kMaxN = 256, kMaxR = 64, kMaxR2 = 64, kMaxClasses = 256, kMaxF = 256;
constexpr double kRmsEps = 1e-6;   // yggdrasil/config.py:8

template <typename T> struct FloatLayerDev {
    const T *table;          // token layer [V][n] (T_x[x]); routed [E][V][n]
    const T *A;              // [E][n/b][b][b] or null
    const T *P;              // [E][R][n]
    const T *Q;              // [classes][R]
    const T *emb;            // routed: [V][F]
    const T *W;              // routed: [nodes][F + n] (router_state) or [nodes][F]
    const T *bias;           // routed: [nodes]
    const T *Vd;             // [R2][n] or null
    const T *Up;             // [E][n][R2] or null
};

template <typename T> struct FloatDevModel {
    int L, n, b, V, classes, D, R, R2, F, router_state;
    const T *output_bias;    // [classes]
    uint32_t *err;
    FloatLayerDev<T> layers[YGG_MAX_LAYERS];
};

template <typename T> __device__ __forceinline__ T wave_sum(T v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <typename T> __device__ __forceinline__ T wave_max(T v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o));
    return v;
}

// atomic max of a non-negative double (its bit pattern orders as an unsigned integer)
__device__ __forceinline__ void atomic_max_nonneg(double *p, double v) {
    atomicMax((unsigned long long *)p, (unsigned long long)__double_as_longlong(v));
}

// stats (calibration maxima, cpu/export.py:127-153), per layer: [|h|, |V' rms(h_below)|, |P_r h|, |h| per 16
// coordinates (n/16), |P_r h| per row (R)]
template <typename T>
__global__ __launch_bounds__(64) void float_kernel(const FloatDevModel<T> m, const int32_t *__restrict__ tokens,
                                                   int Tn, T *__restrict__ state, T *__restrict__ logits,
                                                   int32_t *__restrict__ leaves, double *__restrict__ stats) {
    __shared__ T hs[YGG_MAX_LAYERS][kMaxN];   // states
    __shared__ T bl[kMaxN];                   // rms(h) of the layer below
    __shared__ T hn[kMaxN];                   // the new state of the current layer
    __shared__ T zl[kMaxR2];
    __shared__ T zs[kMaxR];
    __shared__ double gmax[YGG_MAX_LAYERS][kMaxN / 16];

    const int s = blockIdx.x, lane = threadIdx.x;
    const int L = m.L, n = m.n, b = m.b, V = m.V, C = m.classes, R = m.R, R2 = m.R2, F = m.F;
    T *st = state + (size_t)s * L * n;
    for (int l = 0; l < L; l++)
        for (int i = lane; i < n; i += 64) hs[l][i] = st[(size_t)l * n + i];
    for (int l = 0; l < L; l++)
        for (int g = lane; g < n / 16; g += 64) gmax[l][g] = 0.0;
    double smax[YGG_MAX_LAYERS], vmax[YGG_MAX_LAYERS], zmax[YGG_MAX_LAYERS];
    for (int l = 0; l < L; l++) smax[l] = vmax[l] = zmax[l] = 0.0;
    const int sstride = 3 + n / 16 + R;
    __syncthreads();

    const int32_t *tok = tokens + (size_t)s * Tn;
    for (int t = 0; t < Tn; t++) {
        const int x = __builtin_amdgcn_readfirstlane(tok[t]);
        if (x < 0 || x >= V) {
            if (lane == 0) atomicOr(m.err, 1u);
            break;
        }
        T lg[kMaxClasses / 64];
#pragma unroll
        for (int u = 0; u < kMaxClasses / 64; u++) {
            const int c = lane + 64 * u;
            lg[u] = c < C ? m.output_bias[c] : T(0);
        }
        for (int l = 0; l < L; l++) {
            const FloatLayerDev<T> &y = m.layers[l];
            int r = x;
            if (l > 0) {
                // router descent over f = [router_embed[x]; rms(h_below)]
                const T *e = y.emb + (size_t)x * F;
                const int width = F + (m.router_state ? n : 0);
                int node = 0;
                for (int d = 0; d < m.D; d++) {
                    const T *w = y.W + (size_t)node * width;
                    T p = T(0);
                    for (int i = lane; i < width; i += 64) p += (i < F ? e[i] : bl[i - F]) * w[i];
                    p = wave_sum(p) + y.bias[node];
                    node = 2 * node + 1 + (p > T(0) ? 1 : 0);
                }
                r = node - ((1 << m.D) - 1);
            }
            // h = T_r[x] + U'_r (V' rms(h_below)) + A_r h_old
            const T *trow = l == 0 ? y.table + (size_t)x * n : y.table + ((size_t)r * V + x) * n;
            if (l > 0 && y.Vd) {
                if (lane < R2) {
                    T a = T(0);
                    const T *vr = y.Vd + (size_t)lane * n;
                    for (int i = 0; i < n; i++) a += vr[i] * bl[i];
                    zl[lane] = a;
                    vmax[l] = fmax(vmax[l], (double)fabs(a));
                }
                __syncthreads();
            }
            for (int i = lane; i < n; i += 64) {
                T h = trow[i];
                if (l > 0 && y.Up) {
                    const T *u = y.Up + ((size_t)r * n + i) * R2;
                    T a = T(0);
                    for (int k = 0; k < R2; k++) a += u[k] * zl[k];
                    h = h + a;
                }
                if (y.A) {
                    const int g = i / b, ii = i % b;
                    const T *arow = y.A + (((size_t)r * (n / b) + g) * b + ii) * b;
                    T a = T(0);
                    for (int j = 0; j < b; j++) a += arow[j] * hs[l][g * b + j];
                    h = h + a;
                }
                hn[i] = h;
            }
            __syncthreads();
            T ss = T(0);
            double hm = 0.0;
            for (int i = lane; i < n; i += 64) {
                const T h = hn[i];
                hs[l][i] = h;
                ss += h * h;
                hm = fmax(hm, (double)fabs(h));
            }
            smax[l] = fmax(smax[l], hm);
            if (stats)
                for (int g = lane; g < n / 16; g += 64) {
                    double a = 0.0;
                    for (int i = 0; i < 16; i++) a = fmax(a, (double)fabs(hn[16 * g + i]));
                    gmax[l][g] = fmax(gmax[l][g], a);
                }
            // z = P_r h (lane j < R), logits += Q z
            if (lane < R) {
                const T *pr = y.P + ((size_t)r * R + lane) * n;
                T a = T(0);
                for (int i = 0; i < n; i++) a += pr[i] * hn[i];
                zs[lane] = a;
                zmax[l] = fmax(zmax[l], (double)fabs(a));   // lane j holds row j's maximum
            }
            const T rinv = T(1) / sqrt(wave_sum(ss) / T(n) + T(kRmsEps));
            __syncthreads();
            for (int i = lane; i < n; i += 64) bl[i] = hn[i] * rinv;
#pragma unroll
            for (int u = 0; u < kMaxClasses / 64; u++) {
                const int c = lane + 64 * u;
                if (c < C) {
                    const T *q = y.Q + (size_t)c * R;
                    T a = T(0);
                    for (int j = 0; j < R; j++) a += q[j] * zs[j];
                    lg[u] = lg[u] + a;
                }
            }
            if (leaves && lane == 0) leaves[((size_t)s * Tn + t) * L + l] = r;
            __syncthreads();
        }
        if (logits) {
            T *o = logits + ((size_t)s * Tn + t) * C;
#pragma unroll
            for (int u = 0; u < kMaxClasses / 64; u++)
                if (lane + 64 * u < C) o[lane + 64 * u] = lg[u];
        }
    }
    __syncthreads();
    for (int l = 0; l < L; l++)
        for (int i = lane; i < n; i += 64) st[(size_t)l * n + i] = hs[l][i];
    if (stats) {
        for (int l = 0; l < L; l++) {
            const double a = wave_max(smax[l]), v = wave_max(vmax[l]), z = wave_max(zmax[l]);
            if (lane == 0) {
                atomic_max_nonneg(&stats[(size_t)l * sstride + 0], a);
                atomic_max_nonneg(&stats[(size_t)l * sstride + 1], v);
                atomic_max_nonneg(&stats[(size_t)l * sstride + 2], z);
            }
            for (int g = lane; g < n / 16; g += 64) atomic_max_nonneg(&stats[(size_t)l * sstride + 3 + g], gmax[l][g]);
            if (lane < R) atomic_max_nonneg(&stats[(size_t)l * sstride + 3 + n / 16 + lane], zmax[l]);
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
    struct Part { const double *src; int64_t count; size_t off; };
    std::vector<Part> parts;
    size_t total = 256;   // the error word first
    auto add = [&](const double *src, int64_t count) -> int {
        if (!src || count <= 0) return -1;
        parts.push_back({src, count, total});
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
        k.A = add(y.transition, El * n * b);
        k.P = add(y.readout, El * R * n);
        k.Q = add(y.unembed, (int64_t)C * R);
        k.emb = l ? add(y.router_embed, (int64_t)V * F) : -1;
        k.W = l ? add(y.router_weight, nodes * width) : -1;
        k.bias = l ? add(y.router_bias, nodes) : -1;
        k.Vd = (l && R2) ? add(y.layer_input_down, (int64_t)R2 * n) : -1;
        k.Up = (l && R2) ? add(y.layer_input_proj, El * n * R2) : -1;
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
        for (int64_t i = 0; i < p.count; i++) dst[i] = (T)p.src[i];
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
    if (L < 1 || L > YGG_MAX_LAYERS || n < 16 || n > kMaxN || n % 16 || b < 1 || n % b || d->vocab < 1 ||
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
    if (m->precision == 32)
        hipLaunchKernelGGL(float_kernel<float>, dim3(B), dim3(64), 0, (hipStream_t)stream, m->m32, d_tokens, T,
                           (float *)d_state, (float *)d_logits, d_leaves, d_stats);
    else
        hipLaunchKernelGGL(float_kernel<double>, dim3(B), dim3(64), 0, (hipStream_t)stream, m->m64, d_tokens, T,
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
