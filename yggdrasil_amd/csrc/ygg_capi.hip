// C-ABI of the MI355X int8 streaming step: model loading (YGG1 parse, validation, relayout into the device layout of
// ygg_layout.h, upload) and the stream-ordered step/run entry points declared in include/ygg_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/ygg_hip.h"
#include "ygg_launch.h"
#include "ygg_layout.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                                  \
    do {                                                                                               \
        hipError_t e_ = (expr);                                                                        \
        if (e_ != hipSuccess) return fail(YGG_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_));     \
    } while (0)

}  // namespace

// The workspace of ygg_run_grouped_noalloc: one static array per GPU (each device holds its own copy from module
// load until the process ends), shared by every such call on that GPU. Host code uses only the device address
// recorded by scratch_setup, never this name.
static __device__ __align__(256) uint8_t scratch[YGG_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// the address of `scratch` on `device`, which is current: looked up once per device (at the first load onto it)
hipError_t scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return hipSuccess;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = p;
    return hipSuccess;
}

void *scratch_of(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_ptr[device];
}

struct FileArrays {
    int32_t n_layers, n, blk, V, D, R, R2, reserved, router_token_dim, K, shift, n_arrays;
    std::map<std::string, std::pair<const uint8_t *, int64_t>> arr;
    int64_t bytes;
    const uint8_t *get(const std::string &name, int64_t *nb = nullptr) const {
        auto it = arr.find(name);
        if (it == arr.end()) return nullptr;
        if (nb) *nb = it->second.second;
        return it->second.first;
    }
};

// Header + array table (cpu/ygg.cpp:137-171); LIMITS of the reference plus d_state 96.
int parse(const uint8_t *data, size_t size, FileArrays &fa) {
    if (size < 52 || memcmp(data, "YGG1", 4)) return fail(YGG_ERR_FORMAT, "not a model file");
    int32_t h[12];
    memcpy(h, data + 4, sizeof h);
    fa.n_layers = h[0]; fa.n = h[1]; fa.blk = h[2]; fa.V = h[3]; fa.D = h[4]; fa.R = h[5]; fa.R2 = h[6];
    fa.reserved = h[7]; fa.router_token_dim = h[8]; fa.K = h[9]; fa.shift = h[10]; fa.n_arrays = h[11];
    const bool ok = (fa.n == 64 || fa.n == 96 || fa.n == 128 || fa.n == 256) && (fa.blk == 8 || fa.blk == 16) &&
                    (fa.R == 8 || fa.R == 16 || fa.R == 32) && fa.R2 >= 0 && fa.R2 <= YGG_MAX_RANK &&
                    fa.R2 % 4 == 0 && fa.n_layers >= 1 && fa.n_layers <= YGG_MAX_LAYERS && fa.V >= 1 &&
                    fa.V <= 256 && fa.D >= 0 && fa.D <= 16 && (fa.n_layers == 1 || fa.D >= 1) && fa.reserved == 0 &&
                    fa.shift >= 1 && fa.shift <= 30 && fa.n_arrays > 0;
    if (!ok) return fail(YGG_ERR_LIMITS, "unsupported model (LIMITS)");
    const size_t tab_end = 52 + (size_t)fa.n_arrays * 48;
    if (size < tab_end) return fail(YGG_ERR_FORMAT, "short array table");
    const size_t base = (tab_end + 63) / 64 * 64;
    if (size < base) return fail(YGG_ERR_FORMAT, "short model file");
    fa.bytes = (int64_t)(size - base);
    for (int i = 0; i < fa.n_arrays; i++) {
        char name[33] = {0};
        int64_t off, nb;
        memcpy(name, data + 52 + (size_t)i * 48, 32);
        memcpy(&off, data + 52 + (size_t)i * 48 + 32, 8);
        memcpy(&nb, data + 52 + (size_t)i * 48 + 40, 8);
        if (off < 0 || nb < 0 || off > fa.bytes || nb > fa.bytes - off)
            return fail(YGG_ERR_FORMAT, "short model file (array %s)", name);
        fa.arr[name] = {data + base + off, nb};
    }
    return YGG_OK;
}

// Layout sizes of one layer's gather record (see ygg_layout.h).
struct GatherLayout {
    int64_t bytes;
    int off_P, off_U, off_F, off_FB, off_FS;
};
GatherLayout gather_layout(int n, int blk, int R, int R2, int K, bool routed, bool factored) {
    GatherLayout g;
    int64_t o = (int64_t)n * blk * 2;  // A
    g.off_P = (int)o;
    o += (int64_t)R * n;
    g.off_U = -1;
    if (routed && R2) { g.off_U = (int)o; o += (int64_t)R2 * n; }
    g.off_F = g.off_FB = g.off_FS = -1;
    if (factored) {
        g.off_F = (int)o; o += (int64_t)K * n;
        g.off_FB = (int)o; o += 2 * (int64_t)n;
        g.off_FS = (int)o; o += 4;
    }
    g.bytes = (o + 127) / 128 * 128;
    return g;
}

// One file layer's views.
struct FileLayer {
    const uint8_t *rec = nullptr; int64_t rec_nb = 0;
    int record_bytes = 0, off_A = -1, off_U2 = -1, off_P = -1, off_T = -1, off_F = -1, off_C = -1, off_S = -1;
    const uint8_t *Q = nullptr; int64_t Q_nb = 0;
    const float *scal = nullptr;
    const uint8_t *w = nullptr; int64_t w_nb = 0;
    const float *thr = nullptr; int64_t thr_nb = 0;
    const uint8_t *vl = nullptr; int64_t vl_nb = 0;
    const float *mv = nullptr; int64_t mv_nb = 0;
    const float *mulv = nullptr, *r2b = nullptr, *mzl = nullptr, *sqv = nullptr, *mT = nullptr;
    int64_t mulv_nb = 0, r2b_nb = 0, mzl_nb = 0, sqv_nb = 0, mT_nb = 0;
    const int8_t *vt = nullptr; int64_t vt_nb = 0;
};

bool all_finite(const float *p, int64_t count) {
    for (int64_t i = 0; i < count; i++) {
        float v;
        memcpy(&v, p + i, 4);
        if (!std::isfinite(v)) return false;
    }
    return true;
}

// Binds and size-checks the arrays of layer l (cpu/ygg.cpp:173-202); every array the kernels read is checked to hold
// the bytes the kernels will read, so a malformed file fails here instead of faulting on the GPU.
int bind_layer(const FileArrays &fa, int l, FileLayer &y) {
    const std::string P = "l" + std::to_string(l) + "_";
    const int n = fa.n, V = fa.V, E = l == 0 ? fa.V : (1 << fa.D), R = fa.R, R2 = fa.R2;
    const int VP = (V + 31) / 32 * 32;
    int64_t nb = 0;
    auto need = [&](const char *tag, int64_t want, int64_t *got) -> const uint8_t * {
        const uint8_t *p = fa.get(P + tag, got);
        if (!p) { fail(YGG_ERR_FORMAT, "model file: missing %s%s", P.c_str(), tag); return nullptr; }
        if (want >= 0 && *got < want) {
            fail(YGG_ERR_FORMAT, "model file: %s%s holds %lld bytes, needs %lld", P.c_str(), tag, (long long)*got,
                 (long long)want);
            return nullptr;
        }
        return p;
    };
    const int32_t *meta = (const int32_t *)need("meta", 20, &nb);
    if (!meta) return YGG_ERR_FORMAT;
    const int nmeta = (int)(nb / 4);
    y.record_bytes = meta[0]; y.off_A = meta[1]; y.off_U2 = meta[2]; y.off_P = meta[3]; y.off_T = meta[4];
    y.vt = (const int8_t *)fa.get(P + "vt", &y.vt_nb);
    const bool routed = l > 0;
    if (y.vt) {
        if (!routed) return fail(YGG_ERR_FORMAT, "model file: factored token layer");
        if (fa.K % 4 || fa.K > YGG_MAX_RANK || fa.K < 4)
            return fail(YGG_ERR_LIMITS, "model file: factored input_rank %d", fa.K);
        if (nmeta < 8) return fail(YGG_ERR_FORMAT, "model file: %smeta lacks the factored offsets", P.c_str());
        y.off_F = meta[5]; y.off_C = meta[6]; y.off_S = meta[7];
        if (y.vt_nb < (int64_t)V * fa.K) return fail(YGG_ERR_FORMAT, "model file: %svt too short", P.c_str());
        if (!(y.mT = (const float *)need("mT", 4LL * n, &y.mT_nb))) return YGG_ERR_FORMAT;
    }
    if (y.record_bytes <= 0) return fail(YGG_ERR_FORMAT, "model file: %smeta record size", P.c_str());
    // the record parts must lie inside a record
    auto part_ok = [&](int off, int64_t len) { return off >= 0 && off + len <= y.record_bytes; };
    if (!part_ok(y.off_A, 2LL * n * fa.blk) || !part_ok(y.off_P, (int64_t)R * n))
        return fail(YGG_ERR_FORMAT, "model file: %smeta offsets", P.c_str());
    if (routed && R2 && !part_ok(y.off_U2, (int64_t)R2 * n))
        return fail(YGG_ERR_FORMAT, "model file: %smeta layer-input offset", P.c_str());
    if (y.vt) {
        if (!part_ok(y.off_F, (int64_t)fa.K * n) || !part_ok(y.off_C, 2LL * n) || !part_ok(y.off_S, 4))
            return fail(YGG_ERR_FORMAT, "model file: %smeta factored offsets", P.c_str());
    } else if (!part_ok(y.off_T, 2LL * n * (routed ? V : 1))) {
        return fail(YGG_ERR_FORMAT, "model file: %smeta table offset", P.c_str());
    }
    if (!(y.rec = need("rec", (int64_t)E * y.record_bytes, &y.rec_nb))) return YGG_ERR_FORMAT;
    if (!(y.Q = need("Q", (int64_t)R * VP, &y.Q_nb))) return YGG_ERR_FORMAT;
    if (!(y.scal = (const float *)need("scal", 16, &nb))) return YGG_ERR_FORMAT;
    y.mzl = (const float *)fa.get(P + "mzl", &y.mzl_nb);
    if (y.mzl && y.mzl_nb < 4LL * E * (R == 8 ? 16 : R)) return fail(YGG_ERR_FORMAT, "model file: %smzl", P.c_str());
    y.sqv = (const float *)fa.get(P + "sqv", &y.sqv_nb);
    if (y.sqv && y.sqv_nb < 4LL * VP) return fail(YGG_ERR_FORMAT, "model file: %ssqv", P.c_str());
    if (routed) {
        if (!(y.w = need("w", (int64_t)E * n, &y.w_nb))) return YGG_ERR_FORMAT;
        if (!(y.thr = (const float *)need("thr", 4LL * V * E, &y.thr_nb))) return YGG_ERR_FORMAT;
        if (R2) {
            const int RG = (R2 + 15) / 16;
            if (!(y.vl = need("vl", 16LL * RG * n, &y.vl_nb))) return YGG_ERR_FORMAT;
            if (!(y.mv = (const float *)need("mv", 4LL * 16 * RG, &y.mv_nb))) return YGG_ERR_FORMAT;
        }
        y.mulv = (const float *)fa.get(P + "mulv", &y.mulv_nb);
        if (y.mulv && y.mulv_nb < 4LL * n) return fail(YGG_ERR_FORMAT, "model file: %smulv", P.c_str());
        y.r2b = (const float *)fa.get(P + "r2b", &y.r2b_nb);
        if (y.r2b && y.r2b_nb < 4LL * (n / 16)) return fail(YGG_ERR_FORMAT, "model file: %sr2b", P.c_str());
    }
    // Every scale must be a finite number: a NaN or infinite scale would turn every logit of the model into NaN or
    // infinity, and a sampler fed such logits has no class to pick. (Thresholds may be infinite: an infinite
    // threshold sends every stream one way at its node.)
    const struct { const char *tag; const float *p; int64_t count; } scales[] = {
        {"scal", y.scal, 4},
        {"mzl", y.mzl, y.mzl ? (int64_t)E * (R == 8 ? 16 : R) : 0},
        {"sqv", y.sqv, y.sqv ? VP : 0},
        {"mv", y.mv, y.mv ? 16LL * ((R2 + 15) / 16) : 0},
        {"mulv", y.mulv, y.mulv ? n : 0},
        {"r2b", y.r2b, y.r2b ? n / 16 : 0},
        {"mT", y.mT, y.mT ? n : 0},
    };
    for (const auto &sc : scales)
        if (!all_finite(sc.p, sc.count))
            return fail(YGG_ERR_FORMAT, "model file: %s%s holds a scale that is not finite", P.c_str(), sc.tag);
    if (y.vt)
        for (int64_t e = 0; e < E; e++) {
            float v;
            memcpy(&v, y.rec + e * y.record_bytes + y.off_S, 4);
            if (!std::isfinite(v))
                return fail(YGG_ERR_FORMAT, "model file: %srec expert %lld has a factored scale that is not finite",
                            P.c_str(), (long long)e);
        }
    return YGG_OK;
}

inline int16_t rd16(const uint8_t *p) { int16_t v; memcpy(&v, p, 2); return v; }

// Router descent plan (ygg_layout.h): min(4, D) levels, then the rest in ceil(rest / 4) near-equal rounds, larger
// first; YGG_ROUNDS=greedy takes 4 levels per round instead.
struct RoundPlan {
    int n = 0, h[YGG_MAX_ROUNDS] = {0};
};
RoundPlan round_plan(int D) {
    RoundPlan p;
    if (D <= 0) return p;
    const char *env = getenv("YGG_ROUNDS");
    const bool greedy = env && !strcmp(env, "greedy");
    const int h0 = std::min(4, D);
    p.h[p.n++] = h0;
    int rest = D - h0;
    const int nr = (rest + 3) / 4;
    for (int r = 0; r < nr; r++) {
        const int h = greedy ? std::min(4, rest) : (D - h0) / nr + (r < (D - h0) % nr ? 1 : 0);
        p.h[p.n++] = h;
        rest -= h;
    }
    return p;
}

// Slots per token of the round-blocked router arrays: sum over rounds of 2^(d0 + h).
int64_t plan_slots(const RoundPlan &p) {
    int64_t ts = 0;
    int d0 = 0;
    for (int r = 0; r < p.n; r++) { ts += (int64_t)1 << (d0 + p.h[r]); d0 += p.h[r]; }
    return ts;
}

// Visit every (slot, heap node) of the plan; slots with no node (the last of each block) get node -1.
template <class F> void for_each_slot(const RoundPlan &p, F f) {
    int64_t base = 0;
    int d0 = 0;
    for (int r = 0; r < p.n; r++) {
        const int h = p.h[r], bf = 1 << h;
        for (int64_t sub = 0; sub < ((int64_t)1 << d0); sub++) {
            const int64_t ix = ((int64_t)1 << d0) + sub;
            for (int j = 0; j < bf; j++) {
                if (j == bf - 1) { f(base + sub * bf + j, (int64_t)-1); continue; }
                const int dj = 31 - __builtin_clz((unsigned)(j + 1));
                f(base + sub * bf + j, (ix << dj) + (j + 1 - (1 << dj)));
            }
        }
        base += (int64_t)bf << d0;
        d0 += h;
    }
}

// file thr [V][E] (heap order) -> [V][slots] blocked by round and subtree
void block_thresholds(const float *thr, int V, int D, const RoundPlan &p, float *out) {
    const int64_t E = (int64_t)1 << D, ts = plan_slots(p);
    for (int x = 0; x < V; x++) {
        const float *src = thr + (size_t)x * E;
        float *dst = out + (size_t)x * ts;
        for_each_slot(p, [&](int64_t slot, int64_t node) { dst[slot] = node < 0 ? 0.0f : src[node]; });
    }
}

// file w [E][n] u8 (w + 128, heap order) -> [slots][n] s8 blocked by round and subtree
void block_rows(const uint8_t *w, int n, const RoundPlan &p, int8_t *out) {
    for_each_slot(p, [&](int64_t slot, int64_t node) {
        int8_t *dst = out + (size_t)slot * n;
        if (node < 0) { memset(dst, 0, (size_t)n); return; }
        for (int i = 0; i < n; i++) dst[i] = (int8_t)((int)w[(size_t)node * n + i] - 128);
    });
}

template <class F> void parallel_for(int64_t count, F f) {
    int nt = (int)std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()), 16);
    if (count < 256) nt = 1;
    std::vector<std::thread> th;
    for (int k = 0; k < nt; k++)
        th.emplace_back([=]() {
            for (int64_t i = count * k / nt; i < count * (k + 1) / nt; i++) f(i);
        });
    for (auto &t : th) t.join();
}

// A16 = 256 hi + lo with hi, lo signed bytes: lo = ((v + 128) mod 256) - 128, hi = (v - lo) / 256; it exists for
// every v <= 32639
inline int8_t split_lo(int v) { return (int8_t)(((v + 128) & 255) - 128); }
inline int8_t split_hi(int v) { return (int8_t)((v - split_lo(v)) / 256); }

// Does every transition entry of every layer split into signed bytes (the specialised kernels need it)?
bool transitions_split(const FileArrays &fa, const std::vector<FileLayer> &fl) {
    std::atomic<bool> ok{true};
    const int n = fa.n, blk = fa.blk;
    for (size_t l = 0; l < fl.size() && ok; l++) {
        const FileLayer &y = fl[l];
        const int64_t E = l == 0 ? fa.V : ((int64_t)1 << fa.D);
        parallel_for(E, [&](int64_t e) {
            const uint8_t *A = y.rec + e * y.record_bytes + y.off_A;
            for (int64_t k = 0; k < (int64_t)n * blk; k++)
                if (rd16(A + 2 * k) > 32639) { ok = false; return; }
        });
    }
    return ok;
}

// File record of one expert -> its gather record (layout in ygg_layout.h). split: A16 rows as hi bytes then lo bytes.
void relayout_expert(const FileArrays &fa, const FileLayer &fy, const GatherLayout &gl, bool routed, bool split,
                     const uint8_t *frec, uint8_t *g) {
    const int n = fa.n, blk = fa.blk, R = fa.R, R2 = fa.R2, K = fa.K;
    const int C = lanes_c(n), NL = n / C;
    // A: lane l's rows C l .. C l + C - 1, each its b block columns; file [n/16][b/2][16][2] int16
    const uint8_t *A = frec + fy.off_A;
    for (int l = 0; l < NL; l++)
        for (int c = 0; c < C; c++) {
            const int i = C * l + c, g16 = i / 16, rr = i % 16;
            for (int j = 0; j < blk; j++) {
                const int16_t v = rd16(A + (((size_t)(g16 * (blk / 2) + j / 2) * 16 + rr) * 2 + (j & 1)) * 2);
                if (split) {
                    const int hb = c * 2 * blk + j, lb = hb + blk;
                    g[((size_t)(hb / 16) * NL + l) * 16 + hb % 16] = (uint8_t)split_hi(v);
                    g[((size_t)(lb / 16) * NL + l) * 16 + lb % 16] = (uint8_t)split_lo(v);
                } else {
                    const int byte = (c * blk + j) * 2, chunk = byte / 16, within = byte % 16;
                    memcpy(g + ((size_t)chunk * NL + l) * 16 + within, &v, 2);
                }
            }
        }
    // P: lane l -> row j = l / RL, coordinates [(l % RL) SP, +SP); file R = 8: [n/8][16][4], R >= 16: [R/16][n/4][16][4]
    const uint8_t *Pf = frec + fy.off_P;
    const int RL = 64 / R, SP = n / RL, GP = readout_gp(SP);
    for (int l = 0; l < 64; l++) {
        const int j = l / RL, k = l % RL;
        for (int b = 0; b < SP; b++) {
            const int i = k * SP + b;
            size_t o;
            if (R == 8) o = ((size_t)(i / 8) * 16 + 2 * j + (i % 8) / 4) * 4 + i % 4;
            else o = (((size_t)(j / 16) * (n / 4) + i / 4) * 16 + j % 16) * 4 + i % 4;
            g[gl.off_P + ((size_t)(b / GP) * 64 + l) * GP + b % GP] = (uint8_t)((int)Pf[o] - 128);
        }
    }
    // U' and U: file [rank/4][n][4] u8 -> (k4, lane, c) dwords
    auto proj = [&](const uint8_t *src, int rank, int off) {
        for (int k4 = 0; k4 < rank / 4; k4++)
            for (int l = 0; l < NL; l++)
                for (int c = 0; c < C; c++) {
                    const int i = C * l + c;
                    for (int e = 0; e < 4; e++)
                        g[off + (((size_t)k4 * NL + l) * C + c) * 4 + e] =
                            (uint8_t)((int)src[((size_t)k4 * n + i) * 4 + e] - 128);
                }
    };
    if (routed && R2) proj(frec + fy.off_U2, R2, gl.off_U);
    if (gl.off_F >= 0) {
        proj(frec + fy.off_F, K, gl.off_F);
        memcpy(g + gl.off_FB, frec + fy.off_C, 2 * (size_t)n);
        memcpy(g + gl.off_FS, frec + fy.off_S, 4);
    }
}


// every unit of a speculation area to zero (a stale tag)
__global__ void spec_clear_kernel(uint64_t *a, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = 0;
}

}  // namespace

struct DeviceGuard {
    int prev = -1;
    hipError_t set(int dev) {
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) return e;
        return prev == dev ? hipSuccess : hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

struct ygg_model {
    YggDevModel dev;
    ygg_info info;
    int device = 0;
    void *arena = nullptr;
    size_t arena_bytes = 0;
    ygg::Kernel run;                  // per-stream: fast_kernel (4 streams per workgroup, capped) or run_kernel
    ygg::Kernel run_few;              // fast_kernel without the VGPR cap: B <= run_few_max_streams[mode]
    int run_few_max_streams[3] = {0, 0, 0};
    ygg::Kernel pipe;                 // layer-pipelined, 128-VGPR cap: T > 1 and B <= pipe_max_streams
    ygg::Kernel pipe_few;             // the same without the cap: B <= pipe_few_max_streams[mode]
    int pipe_max_streams = 0, pipe_few_max_streams[3] = {0, 0, 0};
    bool pipe_all = false;            // YGG_KERNEL=pipe: every call
    ygg::Kernel deep;                 // deep descent: generate with B <= deep_max_streams
    ygg::Kernel one;                  // the deep descent, second round from global memory: run calls of one token
    int one_max_streams = 0;          // ... with B at most this (its workgroups, one stream each, all resident)
    ygg::Kernel gen_one;              // the same descent for generation past the deep kernel (or without one)
    int gen_one_max_streams = 0;
    int deep_max_streams = 0;
    bool deep_all = false;            // YGG_KERNEL=deep: every call
    ygg::Kernel flow;                 // router rounds and updates pipelined over ticks: T > 1, B <= flow_max_streams[mode]
    int flow_max_streams[3] = {0, 0, 0};
    bool flow_all = false;            // YGG_KERNEL=flow: every call but generation
    ygg::Kernel spec;                 // generation of one stream with speculating helpers (B = 1, T >= 8)
    uint64_t *spec_area = nullptr;    // its speculation area (spec_area_units(V) tagged units)
    mutable uint32_t spec_next = 1;   // the next call's first epoch (epoch 0 never occurs: a cleared unit is stale)
    mutable std::mutex spec_mu;
    int spec_helpers = 0;             // helper workgroups of a call: enough for every candidate token
    bool grouped_ok = false;          // the leaf-grouped step takes the model (ygg_run_grouped)
    void *grp_ws = nullptr;           // its workspace, grown to the largest call
    size_t grp_ws_bytes = 0;
    int grp_mfma_min = 0;             // tiles of at least this many streams on MFMA (0: none)
};

namespace {

int load_impl(const uint8_t *data, size_t size, int device, ygg_model **out) {
    FileArrays fa;
    if (int rc = parse(data, size, fa)) return rc;
    const int L = fa.n_layers, n = fa.n, V = fa.V, VP = (V + 31) / 32 * 32, E = 1 << fa.D, R = fa.R, R2 = fa.R2;
    ygg::Kernel launch = ygg::find_launcher(n, fa.blk, R);
    if (!launch) return fail(YGG_ERR_LIMITS, "no kernel for d_state %d, block %d, readout rank %d", n, fa.blk, R);
    int64_t hb_nb = 0;
    const float *head_b = (const float *)fa.get("head_b", &hb_nb);
    if (!head_b) return fail(YGG_ERR_FORMAT, "missing head_b");
    if (hb_nb < 4LL * VP) return fail(YGG_ERR_FORMAT, "head_b too short");
    if (!all_finite(head_b, VP)) return fail(YGG_ERR_FORMAT, "model file: head_b holds a bias that is not finite");
    std::vector<FileLayer> fl(L);
    bool factored = false, group = false;
    for (int l = 0; l < L; l++) {
        if (int rc = bind_layer(fa, l, fl[l])) return rc;
        factored = factored || fl[l].vt;
        group = group || fl[l].mzl || fl[l].sqv || fl[l].r2b || fl[l].mulv;
    }
    for (int l = 1; l < L; l++)
        if ((fl[l].vt != nullptr) != (fl[1].vt != nullptr))
            return fail(YGG_ERR_FORMAT, "model file: mixed table and factored routed layers");
    // the specialised kernels cover the common shape: fast_kernel for many streams; flow_kernel (one wavefront per
    // layer, router rounds and updates pipelined over ticks), else pipe_kernel (one wavefront per layer), when a call
    // of T > 1 tokens has its B L wavefronts resident at once; generation for few streams on fast_kernel with one
    // stream per workgroup and the deep router descent. YGG_KERNEL=generic|fast|pipe|deep|flow forces one for every
    // call it can run; YGG_DEEP=0 turns the deep descent off, YGG_FLOW=0 flow_kernel.
    const char *kenv = getenv("YGG_KERNEL");
    const std::string kmode = kenv ? kenv : "";
    ygg::Kernel fast;
    // (a shape of YGG_SHAPES, up to 5 layers, group scales at n of 64, 128 or 256; a one-layer model has no layer
    // input and runs at any layer-input rank as 16; every routed layer's table and gather records addressable in 32
    // bits)
    auto shape_ok = [](int nn, int rr, int r2) {
#define YGG_S(N_, R_, R2_) \
    if (nn == N_ && rr == R_ && r2 == R2_) return true;
        YGG_SHAPES(YGG_S)
#undef YGG_S
        return false;
    };
    auto extra_ok = [](int nn, int rr, int r2, int b) {
#define YGG_X(N_, R_, R2_, B_) \
    if (nn == N_ && rr == R_ && r2 == R2_ && b == B_) return true;
        YGG_FAST_EXTRA(YGG_X)
#undef YGG_X
        return false;
    };
    const int R2f = L == 1 ? 16 : R2;
    // std_shape: every specialised kernel family has builds; extra: the per-stream kernel only (YGG_FAST_EXTRA)
    const bool std_shape = fa.blk == 16 && shape_ok(n, R, R2f);
    auto fact_extra_ok = [](int nn, int rr, int r2, int b) {
#define YGG_X(N_, R_, R2_, B_) \
    if (nn == N_ && rr == R_ && r2 == R2_ && b == B_) return true;
        YGG_FACT_EXTRA(YGG_X)
#undef YGG_X
        return false;
    };
    const bool extra_shape = !std_shape && L > 1 &&
                             (factored ? fact_extra_ok(n, R, R2, fa.blk) : extra_ok(n, R, R2, fa.blk));
    const int64_t rec_bound = (int64_t)n * (2 * fa.blk + R2 + R) + 128 +   // gather record bytes, at most
                              (factored ? (int64_t)fa.K * n + 2 * n + 4 : 0);
    const bool small_tables = (int64_t)E * V * n * 2 < ((int64_t)1 << 32) && (int64_t)E * rec_bound < ((int64_t)1 << 32);
    // (factored routed inputs: fact_kernel, input ranks up to 64; the other specialised kernels take table storage)
    if (kmode != "generic" && (std_shape || extra_shape) && L <= ygg::kMaxFastLayers && VP <= 256 &&
        small_tables && (!factored || fa.K <= YGG_MAX_FACT_RANK) && transitions_split(fa, fl))
        fast = extra_shape ? ygg::find_fast_extra_launcher(n, R, R2, fa.blk, L, group, factored)
               : factored  ? ygg::find_fact_launcher(n, R, R2f, L, true, group)
                           : ygg::find_fast_launcher(n, R, R2f, L, true, group);
    if (fast) launch = fast;
    // the other specialised families (deep descent, layer and tick pipelines, grouped) at YGG_SHAPES only
    const bool family = fast && std_shape;

    RoundPlan rplan = round_plan(L > 1 ? fa.D : 0);
    // YGG_ROUNDS=h0,h1,...: an explicit plan for the specialised kernels (every round 1..4 levels, sum D)
    if (const char *rs = getenv("YGG_ROUNDS"); rs && fast && L > 1 && strchr(rs, ',')) {
        RoundPlan p;
        int sum = 0;
        bool ok = true;
        for (const char *c = rs; *c && p.n < YGG_MAX_ROUNDS;) {
            const int h = atoi(c);
            ok = ok && h >= 1 && h <= 4;
            p.h[p.n++] = h;
            sum += h;
            c = strchr(c, ',');
            if (!c) break;
            c++;
        }
        if (!ok || sum != fa.D) return fail(YGG_ERR_ARG, "YGG_ROUNDS=%s: not a plan for depth %d", rs, fa.D);
        rplan = p;
    }
    // the deep descent: at most 4 rounds, the first of at least 2 levels, the rounds after the second at most 6
    // levels together (one lane per node)
    const char *denv = getenv("YGG_DEEP");
    const bool deep = family && !factored && L > 1 && !(denv && !strcmp(denv, "0")) && rplan.n >= 2 && rplan.n <= 4 &&
                      rplan.h[0] >= 2 && (rplan.n < 4 || rplan.h[2] + rplan.h[3] <= 6);
    ygg::Kernel pipe, pipe_few, deepk, flowk;
    if (family && !factored && kmode != "fast" && kmode != "deep" && kmode != "flow") {
        pipe = ygg::find_pipe_launcher(n, R, R2f, L, true, group);
        pipe_few = ygg::find_pipe_launcher(n, R, R2f, L, false, group);
    }
    // the tick-pipelined kernel: plans of 3 or 4 rounds (YGG_FLOW=0: off)
    const char *fenv = getenv("YGG_FLOW");
    if (family && !factored && L > 1 && (kmode == "" || kmode == "flow") && !(fenv && !strcmp(fenv, "0")))
        flowk = ygg::find_flow_launcher(n, R, R2f, L, rplan.n, group);
    // (the deep kernel exists where its LDS fits a workgroup)
    const ygg::Kernel deep_avail = deep ? ygg::find_deep_launcher(n, R, R2f, L, group) : ygg::Kernel();
    if (kmode != "fast" && kmode != "pipe" && kmode != "flow") deepk = deep_avail;
    const int64_t slots = plan_slots(rplan);
    // device arena plan: every array 256-byte aligned
    struct Piece { size_t off, bytes; };
    size_t total = 0;
    auto plan = [&](size_t bytes) { Piece p{total, bytes}; total += (bytes + 255) / 256 * 256; return p; };
    const Piece p_err = plan(256);
    const Piece p_bias = plan(4 * (size_t)VP);
    struct LayerPlan {
        GatherLayout gl;
        Piece gath, table, w, thr, vl, mv, mulv, r2b, mz, sqv, Q, vt, mT;
    };
    std::vector<LayerPlan> lp(L);
    for (int l = 0; l < L; l++) {
        const FileLayer &y = fl[l];
        const bool routed = l > 0;
        const int El = routed ? E : V;
        LayerPlan &p = lp[l];
        p.gl = gather_layout(n, fa.blk, R, R2, fa.K, routed, y.vt != nullptr);
        p.gath = plan((size_t)El * p.gl.bytes);
        p.table = y.vt ? Piece{0, 0} : plan(2 * (size_t)n * (routed ? (size_t)E * V : (size_t)V));
        p.Q = plan((size_t)VP * R);
        // (models with group scales get the array in every layer, holding the layer's scale where the file has none:
        // the kernels then read a row scale without a branch)
        p.mz = (y.mzl || group) ? plan(4 * (size_t)El * R) : Piece{0, 0};
        p.sqv = y.sqv ? plan(4 * (size_t)VP) : Piece{0, 0};
        if (routed) {
            p.w = plan((size_t)slots * n);
            p.thr = plan(4 * (size_t)V * slots);
            const int RG = (R2 + 15) / 16;
            p.vl = R2 ? plan(16 * (size_t)RG * n) : Piece{0, 0};
            p.mv = R2 ? plan(4 * 16 * (size_t)RG) : Piece{0, 0};
            p.mulv = y.mulv ? plan(4 * (size_t)n) : Piece{0, 0};
            p.r2b = y.r2b ? plan(4 * (size_t)(n / 16)) : Piece{0, 0};
            p.vt = y.vt ? plan((size_t)V * fa.K) : Piece{0, 0};
            p.mT = y.vt ? plan(4 * (size_t)n) : Piece{0, 0};
        }
    }
    // host image of the arena
    std::vector<uint8_t> host;
    try {
        host.assign(total, 0);
    } catch (const std::bad_alloc &) {
        return fail(YGG_ERR_NOMEM, "out of host memory (%zu bytes)", total);
    }
    uint8_t *H = host.data();
    memcpy(H + p_bias.off, head_b, 4 * (size_t)VP);
    for (int l = 0; l < L; l++) {
        const FileLayer &y = fl[l];
        const LayerPlan &p = lp[l];
        const bool routed = l > 0;
        const int El = routed ? E : V;
        uint8_t *gath = H + p.gath.off;
        const GatherLayout gl = p.gl;
        const bool split = static_cast<bool>(fast);
        parallel_for(El, [&, gath, gl, routed, split](int64_t e) {
            relayout_expert(fa, y, gl, routed, split, y.rec + e * y.record_bytes, gath + e * gl.bytes);
        });
        if (!y.vt) {
            int16_t *tb = (int16_t *)(H + p.table.off);
            if (routed) {
                parallel_for(E, [&, tb](int64_t e) {
                    memcpy(tb + (size_t)e * V * n, y.rec + e * y.record_bytes + y.off_T, 2 * (size_t)V * n);
                });
            } else {
                for (int x = 0; x < V; x++) memcpy(tb + (size_t)x * n, y.rec + (size_t)x * y.record_bytes + y.off_T, 2 * (size_t)n);
            }
        }
        int8_t *Qd = (int8_t *)(H + p.Q.off);
        for (int c = 0; c < VP; c++)
            for (int j = 0; j < R; j++) Qd[(size_t)c * R + j] = (int8_t)((int)y.Q[((size_t)(j / 4) * VP + c) * 4 + j % 4] - 128);
        if (y.mzl) {
            float *mz = (float *)(H + p.mz.off);
            const int W = R == 8 ? 16 : R;
            for (int e = 0; e < El; e++)
                for (int j = 0; j < R; j++) mz[(size_t)e * R + j] = y.mzl[(size_t)e * W + (R == 8 ? 2 * j : j)];
        } else if (group) {
            float *mz = (float *)(H + p.mz.off);
            for (size_t i = 0; i < (size_t)El * R; i++) mz[i] = y.scal[0];
        }
        if (y.sqv) memcpy(H + p.sqv.off, y.sqv, 4 * (size_t)VP);
        if (routed) {
            block_rows(y.w, n, rplan, (int8_t *)(H + p.w.off));
            block_thresholds(y.thr, V, fa.D, rplan, (float *)(H + p.thr.off));
            if (R2) {
                const int RG = (R2 + 15) / 16;
                int8_t *vd = (int8_t *)(H + p.vl.off);
                for (int k = 0; k < 16 * RG; k++)
                    for (int i = 0; i < n; i++)
                        vd[(size_t)k * n + i] =
                            (int8_t)((int)y.vl[(((size_t)(k / 16) * (n / 4) + i / 4) * 16 + k % 16) * 4 + i % 4] - 128);
                memcpy(H + p.mv.off, y.mv, 4 * 16 * (size_t)RG);
            }
            if (y.mulv) memcpy(H + p.mulv.off, y.mulv, 4 * (size_t)n);
            if (y.r2b) memcpy(H + p.r2b.off, y.r2b, 4 * (size_t)(n / 16));
            if (y.vt) {
                memcpy(H + p.vt.off, y.vt, (size_t)V * fa.K);
                memcpy(H + p.mT.off, y.mT, 4 * (size_t)n);
            }
        }
    }

    // upload: the device is checked only now, so a malformed file is reported as such on any host
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return fail(YGG_ERR_DEVICE, "no HIP device");
    if (device < 0 || device >= count) return fail(YGG_ERR_ARG, "device %d out of range [0, %d)", device, count);
    int prev = 0;
    HIP_TRY(hipGetDevice(&prev));
    HIP_TRY(hipSetDevice(device));
    hipError_t e = scratch_setup(device);
    if (e != hipSuccess) {
        (void)hipSetDevice(prev);
        return fail(YGG_ERR_DEVICE, "the address of the static grouped workspace on device %d: %s", device,
                    hipGetErrorString(e));
    }
    void *arena = nullptr;
    e = hipMalloc(&arena, total);
    if (e != hipSuccess) {
        (void)hipSetDevice(prev);
        return fail(YGG_ERR_NOMEM, "device allocation of %zu bytes failed: %s", total, hipGetErrorString(e));
    }
    e = hipMemcpy(arena, H, total, hipMemcpyHostToDevice);
    (void)hipSetDevice(prev);
    if (e != hipSuccess) {
        (void)hipFree(arena);
        return fail(YGG_ERR_DEVICE, "upload failed: %s", hipGetErrorString(e));
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) cus = 256;
    ygg_model *m = new ygg_model();
    // pipe_kernel when the workgroups of all B streams of a call are resident at once (without the VGPR cap while
    // they fit so), or always with YGG_KERNEL=pipe
    m->pipe = pipe;
    m->pipe_few = pipe_few;
    m->pipe_all = pipe && kmode == "pipe";
    m->pipe_max_streams =
        pipe ? (m->pipe_all ? INT32_MAX : ygg::pipe_blocks_per_cu(n, R, R2f, L, true, group, kModeRun) * cus) : 0;
    // (the uncapped builds per mode: the run build, without the NLL's registers, may keep as many resident as the
    // capped one)
    for (int md : {kModeRun, kModeScore})
        m->pipe_few_max_streams[md] = pipe_few ? ygg::pipe_blocks_per_cu(n, R, R2f, L, false, group, md) * cus : 0;
    // generation with one stream per workgroup while the streams do not outnumber the CUs (for more, the 4 streams
    // per workgroup of fast_kernel win); YGG_KERNEL=deep takes it for every call
    m->deep = deepk;
    m->deep_all = deepk && kmode == "deep";
    // one-token run calls (ygg_step): the deep descent without staging its second round (three dependent global
    // loads per routed layer instead of four) where the deep descent is on and no kernel is forced, one stream per
    // workgroup while the workgroups are all resident (configuration 4: 10.4-13.7 us per step at 4 to 768 streams,
    // against 13.6-14.3 with 4 streams per workgroup, whose tail rounds share a CU's memory path, and 13.3-14.4 on
    // the per-stream run build from 320 streams; past residency, at 1024, the run build: 15.0 against 17.8)
    if (deep && kmode == "") m->one = ygg::find_one_launcher(n, R, R2f, L, group);
    m->one_max_streams = m->one ? ygg::one_blocks_per_cu(n, R, R2f, L, group, false) * cus : 0;
    // generation of more streams than the deep kernel takes (one workgroup per CU), or where no deep kernel fits
    // (its second-round rows beside the tables exceed a workgroup's LDS): the one-token build's descent in a generate
    // build, one stream per workgroup, while its workgroups are all resident (configuration 4 at 257 / 384 / 512
    // streams: 7.4 / 8.0 / 8.0 us per token step against 9.0 / 8.8 / 8.8 on the per-stream generate build)
    if (deep && kmode == "") m->gen_one = ygg::find_gen_one_launcher(n, R, R2f, L, group);
    m->gen_one_max_streams = m->gen_one ? ygg::one_blocks_per_cu(n, R, R2f, L, group, true) * cus : 0;
    // generation of one stream with helper workgroups that compute the next step's first layers for every candidate
    // token (YGG_SPEC=0: off): its speculation area is allocated and cleared here
    const char *spenv = getenv("YGG_SPEC");
    if (deep && kmode == "" && !(spenv && !strcmp(spenv, "0"))) m->spec = ygg::find_spec_launcher(n, R, R2f, L, group);
    m->deep_max_streams = deepk ? (m->deep_all ? INT32_MAX : cus) : 0;
    // flow_kernel for T >= kFlowMinTokens up to flow_max_streams (or always with YGG_KERNEL=flow): measured at 512
    // tokens against the per-stream kernel, the builds with the split descent win up to 8 streams per CU on every
    // benchmark and reference model whether the workgroups are all resident or not (configuration 4's model at 1024
    // streams: 2.30 against 4.54 ms; at 16 per CU the two tie or the per-stream kernel wins), the unsplit build of the
    // largest shape up to two rounds of resident workgroups (per mode: the 5-layer score builds are unsplit, and the
    // largest shape's has one wavefront more; generation never runs on it)
    m->flow = flowk;
    m->flow_all = flowk && kmode == "flow";
    for (int md : {kModeRun, kModeScore}) {
        const int resident = flowk ? ygg::flow_blocks_per_cu(n, R, R2f, L, rplan.n, group, md) * cus : 0;
        const int reach = ygg::flow_split_build(n, R, R2f, L, md) ? 8 * cus : 2 * resident;
        m->flow_max_streams[md] = flowk ? (m->flow_all ? INT32_MAX : std::max(resident, reach)) : 0;
    }
    // the leaf-grouped step: the benchmark shape with the specialised kernels' record layout, tensor scales, tables
    m->grouped_ok = family && !factored && !group && n == 128 && R == 8 && R2f == 16 && fa.blk == 16 &&
                    (L == 1 || fa.D <= 14);
    {
        const char *gm = getenv("YGG_GROUP_MFMA_MIN");
        m->grp_mfma_min = gm ? atoi(gm) : 8;
    }
    m->device = device;
    m->arena = arena;
    m->arena_bytes = total;
    if (m->spec) {
        // (without it, generation runs without helpers)
        DeviceGuard sg;
        void *a = nullptr;
        const size_t bytes = spec_area_units(V) * sizeof(uint64_t);
        if (sg.set(device) != hipSuccess || hipMalloc(&a, bytes) != hipSuccess || hipMemset(a, 0, bytes) != hipSuccess ||
            hipDeviceSynchronize() != hipSuccess) {
            if (a) (void)hipFree(a);
            m->spec = ygg::Kernel();
        } else {
            m->spec_area = (uint64_t *)a;
        }
        // helper workgroups, one CU each (the stream's and the helpers' all resident at once), one helper wavefront
        // per candidate token: one per workgroup where the CUs allow, two on as many as needed (spec_pairs); at
        // d_state 256 two on every one (one wavefront per CU: configuration 4 4.63 -> 4.55 us per token, the
        // reference's medium shape 5.26 -> 5.03, its large shape 10.5 -> 10.8); YGG_SPEC_HELPERS: fewer
        m->spec_helpers = std::min(std::min(kSpecMaxHelpers, cus - 1), n > 128 ? (V + 1) / 2 : V);
        if (const char *eh = getenv("YGG_SPEC_HELPERS")) m->spec_helpers = std::max(0, std::min(m->spec_helpers, atoi(eh)));
        // YGG_SPEC_EPOCH: the first call's first epoch (tests of the wrap; 0 is taken as 1)
        if (const char *ep = getenv("YGG_SPEC_EPOCH")) m->spec_next = (uint32_t)strtoul(ep, nullptr, 0);
        if (m->spec_next == 0) m->spec_next = 1;
    }
    m->run = launch;
    // the uncapped per-stream build while every stream of the call is resident with it
    if (family) {
        m->run_few = factored ? ygg::find_fact_launcher(n, R, R2f, L, false, group)
                              : ygg::find_fast_launcher(n, R, R2f, L, false, group);
        for (int md = 0; md < 3; md++)
            m->run_few_max_streams[md] = (factored ? ygg::fact_blocks_per_cu(n, R, R2f, L, false, group, md)
                                                   : ygg::fast_blocks_per_cu(n, R, R2f, L, false, group, md)) *
                                         4 * cus;
    }
    uint8_t *A = (uint8_t *)arena;
    auto at = [&](const Piece &p) -> void * { return p.bytes ? A + p.off : nullptr; };
    YggDevModel &d = m->dev;
    d.L = L; d.N = n; d.BLK = fa.blk; d.V = V; d.VP = VP; d.D = fa.D; d.E = E; d.R = R; d.R2 = R2; d.K = fa.K;
    d.shift = fa.shift;
    d.n_rounds = rplan.n;
    d.round_pack = 0;
    for (int r = 0; r < YGG_MAX_ROUNDS; r++) {
        d.round_h[r] = rplan.h[r];
        d.round_pack |= (uint64_t)(rplan.h[r] & 15) << (4 * r);
    }
    d.output_bias = (const float *)at(p_bias);
    d.err = (uint32_t *)at(p_err);
    for (int l = 0; l < L; l++) {
        const FileLayer &y = fl[l];
        const LayerPlan &p = lp[l];
        YggDevLayer &z = d.layers[l];
        z.gath = (const uint8_t *)at(p.gath);
        z.table = (const int16_t *)at(p.table);
        z.w = (const int8_t *)at(p.w);
        z.thr = (const float *)at(p.thr);
        z.vl = (const int8_t *)at(p.vl);
        z.mv = (const float *)at(p.mv);
        z.mulv = (const float *)at(p.mulv);
        z.r2b = (const float *)at(p.r2b);
        z.mz = (const float *)at(p.mz);
        z.sqv = (const float *)at(p.sqv);
        z.Q = (const int8_t *)at(p.Q);
        z.vt = (const int8_t *)at(p.vt);
        z.mT = (const float *)at(p.mT);
        z.gath_bytes = p.gl.bytes;
        z.table_sr = l == 0 ? n : (int64_t)V * n;
        z.table_sx = l == 0 ? 0 : n;
        z.off_P = p.gl.off_P; z.off_U = p.gl.off_U; z.off_F = p.gl.off_F; z.off_FB = p.gl.off_FB;
        z.off_FS = p.gl.off_FS;
        z.thr_stride = l > 0 ? (int32_t)slots : 0;
        z.readout_scale = y.scal[0]; z.unembed_scale = y.scal[1]; z.rms_eps = y.scal[2];
        z.layer_input_scale = y.scal[3];
    }
    ygg_info &I = m->info;
    memset(&I, 0, sizeof I);
    I.n_layers = L; I.d_state = n; I.block_size = fa.blk; I.vocab = V; I.vocab_pad = VP; I.router_depth = fa.D;
    I.n_experts = E; I.readout_rank = R; I.layer_input_rank = R2; I.input_rank = fa.K; I.shift = fa.shift;
    I.factored = factored; I.group = group; I.device = device; I.kernel = fast ? 1 : 0;
    I.pipe_max_streams = m->pipe_max_streams;
    I.deep = deep_avail ? 1 : 0;
    I.deep_max_streams = m->deep_max_streams;
    I.flow_max_streams = m->flow_max_streams[kModeRun];
    I.router_rounds = L > 1 ? rplan.n : 0;
    I.spec_max_streams = m->spec ? 1 : 0;
    I.grouped = m->grouped_ok ? 1 : 0;
    I.file_array_bytes = fa.bytes;
    I.device_bytes = (int64_t)total;
    for (int l = 0; l < L; l++) I.gather_bytes[l] = lp[l].gl.bytes;
    *out = m;
    return YGG_OK;
}

// flow_kernel's pipeline fills over (L - 1)(P + 1) + 2 ticks (up to 17 at 4 layers and 4 rounds): calls of fewer
// tokens run faster on pipe_kernel (measured break-even about 24 tokens on configuration 4's model)
constexpr int kFlowMinTokens = 32;

// The kernel of a call of B streams and T tokens in mode (kModeRun, kModeGenerate: ygg_generate, kModeScore: a
// digest or NLL). Run calls of one token with all their streams resident on the one-token build (one stream per
// workgroup): that build (the deep descent, its second round from global memory). Generation: the deep kernel for
// >= 8 tokens and B <= deep_max_streams, then the generate build with the one-token build's descent while its
// workgroups are all resident, else the per-stream kernel (every token needs all layers of the one before
// it, so never a layer-pipelined one). Otherwise: the tick-pipelined kernel for T >= kFlowMinTokens and B <= flow_max_streams, the layer-pipelined kernel for T > 1 when its
// workgroups fit (for T >= kFlowMinTokens only where there is no tick-pipelined build: more streams than that one
// takes run best on the per-stream kernel), else the per-stream kernel. Of the two builds of a kernel, the uncapped
// one while all B streams are resident with it. A kernel forced by YGG_KERNEL takes every call it can run.
const ygg::Kernel &pick(const ygg_model *m, int B, int T, int mode) {
    const bool gen = mode == kModeGenerate;
    if (m->deep_all) return m->deep;
    if (gen && m->spec && B == 1 && T >= 8) return m->spec;
    if (m->one && mode == kModeRun && T == 1 && B <= m->one_max_streams) return m->one;
    if (gen && m->deep && B <= m->deep_max_streams && T >= 8) return m->deep;
    if (gen && m->gen_one && B <= m->gen_one_max_streams && T >= 8) return m->gen_one;
    if (!gen && m->flow && (m->flow_all || (T >= kFlowMinTokens && B <= m->flow_max_streams[mode]))) return m->flow;
    if (!gen && m->pipe && (m->pipe_all || (T > 1 && B <= m->pipe_max_streams && !(m->flow && T >= kFlowMinTokens))))
        return (m->pipe_few && B <= m->pipe_few_max_streams[mode]) ? m->pipe_few : m->pipe;
    return (m->run_few && B <= m->run_few_max_streams[mode]) ? m->run_few : m->run;
}


}  // namespace

namespace ygg {
// the thread's last error, for the other sources of the library
int set_error(int code, const char *msg) { return fail(code, "%s", msg); }
}  // namespace ygg

extern "C" {

int ygg_version(void) { return 11; }

const char *ygg_last_error(void) { return g_err.c_str(); }

int ygg_load_blob(const void *data, size_t bytes, int device, ygg_model **out) {
    if (!out) return fail(YGG_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (!data) return fail(YGG_ERR_ARG, "data is NULL");
    if (device < 0) return fail(YGG_ERR_ARG, "device %d out of range", device);
    return load_impl((const uint8_t *)data, bytes, device, out);
}

int ygg_load(const char *path, int device, ygg_model **out) {
    if (!out) return fail(YGG_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (!path) return fail(YGG_ERR_ARG, "path is NULL");
    FILE *f = fopen(path, "rb");
    if (!f) return fail(YGG_ERR_IO, "%s: cannot open", path);
    fseek(f, 0, SEEK_END);
    const long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (sz < 0) { fclose(f); return fail(YGG_ERR_IO, "%s: cannot size", path); }
    std::vector<uint8_t> buf;
    try {
        buf.resize((size_t)sz);
    } catch (const std::bad_alloc &) {
        fclose(f);
        return fail(YGG_ERR_NOMEM, "out of host memory (%ld bytes)", sz);
    }
    size_t got = 0;
    while (got < (size_t)sz) {
        const size_t c = fread(buf.data() + got, 1, std::min<size_t>((size_t)sz - got, 64u << 20), f);
        if (!c) break;
        got += c;
    }
    fclose(f);
    if (got != (size_t)sz) return fail(YGG_ERR_IO, "%s: short read", path);
    return ygg_load_blob(buf.data(), buf.size(), device, out);
}

int ygg_model_info(const ygg_model *m, ygg_info *info) {
    if (!m || !info) return fail(YGG_ERR_ARG, "NULL argument");
    *info = m->info;
    return YGG_OK;
}

void ygg_free(ygg_model *m) {
    if (!m) return;
    DeviceGuard g;
    if (g.set(m->device) == hipSuccess) {
        (void)hipFree(m->arena);
        if (m->grp_ws) (void)hipFree(m->grp_ws);
        if (m->spec_area) (void)hipFree(m->spec_area);
    }
    delete m;
}

int ygg_run(const ygg_model *m, const int32_t *d_tokens, int B, int T, int8_t *d_state, float *d_logits,
            int32_t *d_leaves, int8_t *d_states, uint64_t *d_digest, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0 || T < 0) return fail(YGG_ERR_ARG, "negative B (%d) or T (%d)", B, T);
    if (B == 0) return YGG_OK;
    if (!d_state || (T > 0 && !d_tokens)) return fail(YGG_ERR_ARG, "tokens or state is NULL");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    // the pipelined kernel overlaps the layers of consecutive tokens, so it needs more than one token per launch
    const ygg::Kernel &k = pick(m, B, T, d_digest ? kModeScore : kModeRun);
    YggIO io{};
    io.logits = d_logits;
    io.leaves = d_leaves;
    io.states = d_states;
    io.digest = (unsigned long long *)d_digest;
    HIP_TRY(k.fn(m->dev, d_tokens, B, T, d_state, io, (hipStream_t)stream));
    return YGG_OK;
}

int ygg_run_grouped(ygg_model *m, const int32_t *d_tokens, int B, int T, int8_t *d_state, float *d_logits,
                    int32_t *d_leaves, int8_t *d_states, uint64_t *d_digest, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0 || T < 0) return fail(YGG_ERR_ARG, "negative B (%d) or T (%d)", B, T);
    if (!m->grouped_ok)
        return fail(YGG_ERR_LIMITS, "the grouped step takes d_state 128, readout rank 8, layer-input rank 16, block 16, "
                                    "table storage, tensor scales and router depth at most 14");
    if (B == 0 || T == 0) return YGG_OK;
    if (!d_state || !d_tokens) return fail(YGG_ERR_ARG, "tokens or state is NULL");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    const size_t need = ygg::grouped_ws_bytes(B, m->dev.L);
    if (need > m->grp_ws_bytes) {
        // (stream-ordered use of the old workspace ends before it is freed)
        HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
        if (m->grp_ws) (void)hipFree(m->grp_ws);
        m->grp_ws = nullptr;
        m->grp_ws_bytes = 0;
        HIP_TRY(hipMalloc(&m->grp_ws, need));
        m->grp_ws_bytes = need;
    }
    YggIO io{};
    io.logits = d_logits;
    io.leaves = d_leaves;
    io.states = d_states;
    io.digest = (unsigned long long *)d_digest;
    HIP_TRY(ygg::launch_grouped(m->dev, d_tokens, B, T, d_state, io, m->grp_ws, m->grp_mfma_min,
                                (hipStream_t)stream));
    return YGG_OK;
}

int ygg_run_grouped_noalloc(const ygg_model *m, const int32_t *d_tokens, int B, int T, int8_t *d_state,
                            float *d_logits, int32_t *d_leaves, int8_t *d_states, uint64_t *d_digest, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0 || T < 0) return fail(YGG_ERR_ARG, "negative B (%d) or T (%d)", B, T);
    if (!m->grouped_ok)
        return fail(YGG_ERR_LIMITS, "the grouped step takes d_state 128, readout rank 8, layer-input rank 16, block 16, "
                                    "table storage, tensor scales and router depth at most 14");
    if (B == 0 || T == 0) return YGG_OK;
    if (!d_state || !d_tokens) return fail(YGG_ERR_ARG, "tokens or state is NULL");
    const size_t need = ygg::grouped_ws_bytes(B, m->dev.L);
    if (need > (size_t)YGG_SCRATCH_BYTES)
        return fail(YGG_ERR_LIMITS, "ygg_run_grouped_noalloc: %d streams of a %d-layer model need %zu bytes of "
                                    "workspace, more than its static %d (ygg_run_grouped has no such limit)",
                    B, m->dev.L, need, YGG_SCRATCH_BYTES);
    void *ws = scratch_of(m->device);
    if (!ws) return fail(YGG_ERR_DEVICE, "no static grouped workspace on device %d", m->device);
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    YggIO io{};
    io.logits = d_logits;
    io.leaves = d_leaves;
    io.states = d_states;
    io.digest = (unsigned long long *)d_digest;
    HIP_TRY(ygg::launch_grouped(m->dev, d_tokens, B, T, d_state, io, ws, m->grp_mfma_min, (hipStream_t)stream));
    return YGG_OK;
}

int ygg_softmax(const float *d_logits, int64_t rows, int V, float *d_probs, float *d_lse, void *stream) {
    if (rows < 0) return fail(YGG_ERR_ARG, "negative rows (%lld)", (long long)rows);
    if (V < 1 || V > 256) return fail(YGG_ERR_ARG, "V = %d outside [1, 256]", V);
    if (rows == 0) return YGG_OK;
    if (!d_logits || !d_probs) return fail(YGG_ERR_ARG, "logits or probs is NULL");
    HIP_TRY(ygg::launch_softmax(d_logits, rows, V, d_probs, d_lse, (hipStream_t)stream));
    return YGG_OK;
}

int ygg_score(const ygg_model *m, const int32_t *d_tokens, const int32_t *d_targets, int B, int T, int8_t *d_state,
              double *d_nll, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0 || T < 0) return fail(YGG_ERR_ARG, "negative B (%d) or T (%d)", B, T);
    if (B == 0) return YGG_OK;
    if (!d_state || !d_nll || (T > 0 && (!d_tokens || !d_targets))) return fail(YGG_ERR_ARG, "NULL buffer");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    const ygg::Kernel &k = pick(m, B, T, kModeScore);
    YggIO io{};
    io.targets = d_targets;
    io.nll = d_nll;
    HIP_TRY(k.fn(m->dev, d_tokens, B, T, d_state, io, (hipStream_t)stream));
    return YGG_OK;
}

int ygg_generate(const ygg_model *m, const int32_t *d_first, int B, int n, int8_t *d_state, float temperature,
                 int top_k, uint64_t seed, int32_t *d_out, float *d_logits, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0 || n < 0) return fail(YGG_ERR_ARG, "negative B (%d) or n (%d)", B, n);
    if (!(temperature >= 0.0f) || temperature == __builtin_huge_valf())
        return fail(YGG_ERR_ARG, "temperature %g: finite and >= 0", (double)temperature);
    if (top_k < 0) return fail(YGG_ERR_ARG, "negative top_k (%d)", top_k);
    if (B == 0 || n == 0) return YGG_OK;
    if (!d_first || !d_state || !d_out) return fail(YGG_ERR_ARG, "NULL buffer");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    const ygg::Kernel &k = pick(m, B, n, kModeGenerate);
    YggIO io{};
    io.logits = d_logits;
    io.gen = d_out;
    io.temperature = temperature;
    io.top_k = top_k;
    io.seed = (unsigned long long)seed;
    if (&k == &m->spec) {
        // the call's epochs E0 .. E0 + n (a tag of every unit its stream and helpers store); before they would wrap,
        // the area is cleared on the stream and the epochs start again at 1
        std::lock_guard<std::mutex> lk(m->spec_mu);
        if ((uint64_t)m->spec_next + (uint64_t)n + 1 > 0xFFFFFFFFull) {
            const size_t units = spec_area_units(m->dev.V);
            hipLaunchKernelGGL(spec_clear_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                               (hipStream_t)stream, m->spec_area, units);
            HIP_TRY(hipGetLastError());
            m->spec_next = 1;
        }
        io.spec = m->spec_area;
        io.spec_epoch = m->spec_next;
        io.spec_helpers = m->spec_helpers;
        m->spec_next += (uint32_t)n + 1;
    }
    HIP_TRY(k.fn(m->dev, d_first, B, n, d_state, io, (hipStream_t)stream));
    return YGG_OK;
}

int ygg_spec_stats(const ygg_model *m, uint64_t *out, int reset) {
    if (!m || !out) return fail(YGG_ERR_ARG, "NULL argument");
    memset(out, 0, kSpecNStats * sizeof(uint64_t));
    if (!m->spec_area) return YGG_OK;
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    HIP_TRY(hipMemcpy(out, m->spec_area + kSpecStats, kSpecNStats * sizeof(uint64_t), hipMemcpyDeviceToHost));
    if (reset) HIP_TRY(hipMemset(m->spec_area + kSpecStats, 0, kSpecNStats * sizeof(uint64_t)));
    return YGG_OK;
}

int ygg_step(const ygg_model *m, const int32_t *d_tokens, const int8_t *d_state_in, int8_t *d_state_out,
             float *d_logits, int32_t *d_leaves, int B, void *stream) {
    if (!m) return fail(YGG_ERR_ARG, "model is NULL");
    if (B < 0) return fail(YGG_ERR_ARG, "negative B (%d)", B);
    if (B == 0) return YGG_OK;
    if (!d_tokens || !d_state_in || !d_state_out || !d_logits) return fail(YGG_ERR_ARG, "NULL buffer");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    if (d_state_in != d_state_out)
        HIP_TRY(hipMemcpyAsync(d_state_out, d_state_in, (size_t)B * m->dev.L * m->dev.N, hipMemcpyDeviceToDevice,
                               (hipStream_t)stream));
    // one token: a per-stream kernel (a one-token launch cannot overlap layers), or a forced one
    const ygg::Kernel &k = pick(m, B, 1, kModeRun);
    YggIO io{};
    io.logits = d_logits;
    io.leaves = d_leaves;
    HIP_TRY(k.fn(m->dev, d_tokens, B, 1, d_state_out, io, (hipStream_t)stream));
    return YGG_OK;
}

int ygg_kernel_name(const ygg_model *m, int B, int T, int mode, char *name, size_t len) {
    if (!m || !name || len == 0) return fail(YGG_ERR_ARG, "NULL argument");
    if (B < 0 || T < 0) return fail(YGG_ERR_ARG, "negative B (%d) or T (%d)", B, T);
    if (mode < 0 || mode > 2) return fail(YGG_ERR_ARG, "mode %d: 0 run, 1 generate, 2 score or digest", mode);
    pick(m, B, T, mode).name_for(mode, name, len);
    return YGG_OK;
}

int ygg_take_errors(const ygg_model *m, void *stream, uint32_t *errors) {
    if (!m || !errors) return fail(YGG_ERR_ARG, "NULL argument");
    DeviceGuard g;
    HIP_TRY(g.set(m->device));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    uint32_t v = 0;
    HIP_TRY(hipMemcpy(&v, m->dev.err, 4, hipMemcpyDeviceToHost));
    if (v) {
        const uint32_t zero = 0;
        HIP_TRY(hipMemcpy(m->dev.err, &zero, 4, hipMemcpyHostToDevice));
    }
    *errors = v;
    return YGG_OK;
}

}  // extern "C"
