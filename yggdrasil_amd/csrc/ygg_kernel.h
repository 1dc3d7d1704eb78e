// The fused int8 streaming step for gfx950: one 64-lane wavefront per stream, every layer of every token of a
// T-token launch in one kernel, the int8 states of all layers resident in LDS for the whole launch.
//
// Per token and layer (cpu/ygg.cpp:441-459):
//   routed layer   rho from the layer below (per-16-coordinate sums in 16 lanes, cpu/ygg.cpp:248-266); the router
//                  descent in rounds of up to 4 levels (the model's round plan): up to 15 quads take the nodes of
//                  the subtree below the current node, each quad forms one node's dot product (quad lanes split the
//                  coordinates, a DPP quad sum joins them), one ballot of the comparisons gives the whole path
//                  through the subtree in scalar registers (cpu/ygg.cpp:271-280); the layer input zl from V' in the
//                  same quad layout
//                  (cpu/ygg.cpp:285-296)
//   every layer    the expert's gather record (A16, U', P) and its table row are loaded as soon as the expert is
//                  known; transition with v_dot2 (int16 x int16), table or factored input, layer input with v_dot4,
//                  sat8 (cpu/ygg.cpp:311-389); readout P q with v_dot4 and a DPP sum over the lanes of each row,
//                  zq, then the unembedding of 4 classes per lane into the f32 logits (cpu/ygg.cpp:395-435)
//
// f32 arithmetic is one rounded operation per step in the reference's order; the file is compiled with
// -ffp-contract=off, sqrtf is the correctly rounded square root and '/' the correctly rounded division.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ygg_layout.h"

namespace ygg {

typedef short s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
__device__ __forceinline__ int dot2(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), c, false);
}
// DPP sums over 2, 4 and 8 consecutive lanes (every lane of the group gets the sum)
__device__ __forceinline__ int sum2(int v) { return v + __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int sum4(int v) {
    v = sum2(v);
    return v + __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
}
__device__ __forceinline__ int sum8(int v) {
    v = sum4(v);
    return v + __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
}
template <int G> __device__ __forceinline__ int group_sum(int v) {
    if constexpr (G == 1) return v;
    else if constexpr (G == 2) return sum2(v);
    else if constexpr (G == 4) return sum4(v);
    else return sum8(v);
}
__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    for (int o = 32; o >= 1; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o);
    return v;
}

template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// fmaxf over the wavefront (every lane active), returned to every lane: DPP within rows of 16 lanes (quad swaps, the
// half-row and row mirrors), then the four row maxima from scalar reads. fmaxf ignores NaNs and is exact, so the order
// of the pairings does not change the result.
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// The NLL of a stream's scored tokens in double, the reference's score mode (cpu/ygg.cpp:514-516): per token
// mx = max_c lg[c], se = sum_c exp(lg[c] - mx) and the term log(se) + mx - lg[y]. The sum over a stream is kept as
// lin = sum of (mx - lg[y]) and the product of the se (each in [1, V]) as a mantissa pm in [0.5, 1) times 2^pe,
// renormalised exactly (frexp) after every token, so that one log per stream, value(), replaces one per token (whose
// polynomial constants would otherwise stay live through the token loop). The product's rounding adds about one ulp
// of relative error per token to it, a few 1e-14 of absolute error in the log over 1024 tokens.
// a value every lane of the wavefront holds alike, moved to scalar registers (where a per-stream accumulator then stays)
__device__ __forceinline__ unsigned long long uniform_u64(unsigned long long u) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u), hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ double uniform_f64(double v) {
    return __builtin_bit_cast(double, uniform_u64(__builtin_bit_cast(unsigned long long, v)));
}
// (lin, pm and pe are uniform over the wavefront, every lane forming the same sums: kept in scalar registers)
struct NllSum {
    double lin = 0.0, pm = 1.0;
    int pe = 0;
    __device__ __forceinline__ void add(double se, double lin_t) {
        lin = uniform_f64(lin + lin_t);
        int e;
        pm = uniform_f64(frexp(pm * se, &e));
        pe = __builtin_amdgcn_readfirstlane(pe + e);
    }
    __device__ __forceinline__ double value() const { return log(pm) + (double)pe * 0.69314718055994530942 + lin; }
};

// e^d for d <= 0 in double: d = k ln 2 + r with k = rint(d / ln 2), |r| <= ln 2 / 2 (Cody and Waite's reduction: ln 2
// in two parts, the first with 20 significant bits, so that k times it is exact), e^r by its Taylor series to degree
// 13 (the remainder r^14 / 14! stays below 2^-57 of e^r), scaled by 2^k; below -745.5 the result is 0 (e^d is then
// below half the smallest subnormal double). Within one ulp of the C library's exp (checked on the host over 2e7
// arguments in [-800, 0]). The coefficients come from kExpNeg through c, a pointer the caller launders once per call
// (an empty asm), so that they are scalar loads at each call instead of 12 double constants the compiler would keep
// in vector registers through the token loop.
static __constant__ double kExpNeg[14] = {
    1.4426950408889634,                    // 1 / ln 2
    0x1.62e42p-1, 0x1.fdf473de6af28p-22,   // ln 2 = high part + low part
    1.0 / 6227020800.0, 1.0 / 479001600.0, 1.0 / 39916800.0, 1.0 / 3628800.0, 1.0 / 362880.0, 1.0 / 40320.0,
    1.0 / 5040.0, 1.0 / 720.0, 1.0 / 120.0, 1.0 / 24.0, 1.0 / 6.0};   // 1 / j! for j = 13 .. 3
typedef const __attribute__((address_space(4))) double *ConstF64;
__device__ __forceinline__ double exp_neg(double d, ConstF64 c) {
    const double k = rint(d * c[0]);
    double r = fma(-k, c[1], d);
    r = fma(-k, c[2], r);
    double p = c[3];
#pragma unroll
    for (int j = 4; j < 14; j++) p = fma(p, r, c[j]);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    return d < -745.5 ? 0.0 : ldexp(p, (int)k);
}

// Token t's term into acc: lg classes [4 lane, 4 lane + 4) of this lane, V classes; y is uniform and in range. The
// sum over classes runs as a tree over lanes instead of in class order, so se can differ from the reference's in its
// last bits.
__device__ __forceinline__ void token_nll(NllSum &acc, const float (&lg)[4], int V, int y, int lane) {
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < 4; u++)
        if (4 * lane + u < V) mx = fmaxf(mx, lg[u]);
    mx = wave_max_f32(mx);
    ConstF64 c = (ConstF64)kExpNeg;
    asm volatile("" : "+s"(c));
    double se = 0.0;
#pragma unroll
    for (int u = 0; u < 4; u++)
        if (4 * lane + u < V) se += exp_neg((double)lg[u] - (double)mx, c);
    se = wave_sum_f64(se);
    float ly = lg[0];
#pragma unroll
    for (int u = 1; u < 4; u++) ly = (y & 3) == u ? lg[u] : ly;
    ly = __shfl(ly, y >> 2);
    acc.add(se, (double)mx - (double)ly);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
// inclusive prefix sum over lanes
__device__ __forceinline__ float wave_scan_f32(float v, int lane) {
    for (int o = 1; o < 64; o <<= 1) {
        const float u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}
// SplitMix64's output function (Steele, Lea, Flood 2014): a 64-bit mixer for counter-based random numbers
__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// order-preserving map of a float to an unsigned key
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The next token from the logits of one stream (4 classes per lane, V classes; the sampling of
// yggdrasil/inference.py:102-107 and yggdrasil/inference_triton.py:236-242): temperature 0 takes the first maximal
// class; otherwise classes below the top_k-th largest logit are dropped and a class is drawn with probability
// proportional to exp((lg - max) / temperature), by inverse CDF with a uniform from (seed, stream, step).
__device__ __forceinline__ int sample_token(const float (&lg)[4], int V, float temperature, int top_k,
                                            unsigned long long seed, int s, int t, int lane) {
    bool valid[4];
#pragma unroll
    for (int u = 0; u < 4; u++) valid[u] = 4 * lane + u < V;
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < 4; u++)
        if (valid[u]) mx = fmaxf(mx, lg[u]);
    mx = wave_max_f32(mx);
    if (temperature <= 0.0f) {
        // the first maximal class: the lowest lane holding one, then its lowest class (scalar work on ballots)
        unsigned long long mk[4], any = 0;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            mk[u] = __ballot(valid[u] && lg[u] == mx);
            any |= mk[u];
        }
        if (!any) return 0x7fffffff;
        const int ln = __builtin_ctzll(any);
        const int u = ((mk[0] >> ln) & 1) ? 0 : (((mk[1] >> ln) & 1) ? 1 : (((mk[2] >> ln) & 1) ? 2 : 3));
        return 4 * ln + u;
    }
    // the top_k-th largest logit, by a radix search over order-preserving keys
    uint32_t kth = 0;
    if (top_k > 0 && top_k < V) {
        uint32_t key[4];
#pragma unroll
        for (int u = 0; u < 4; u++) key[u] = fkey(lg[u]);
        for (int b = 31; b >= 0; b--) {
            const uint32_t cand = kth | (1u << b);
            int c = 0;     // classes with keys >= cand: population counts of ballots
#pragma unroll
            for (int u = 0; u < 4; u++) c += __popcll(__ballot(valid[u] && key[u] >= cand));
            if (c >= top_k) kth = cand;
        }
    }
    float w[4], part = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const bool keep = valid[u] && fkey(lg[u]) >= kth;
        w[u] = keep ? expf((lg[u] - mx) / temperature) : 0.0f;
        part += w[u];
    }
    const float incl = wave_scan_f32(part, lane);
    const float total = __shfl(incl, 63);
    const unsigned long long r = mix64(seed ^ mix64(((unsigned long long)s << 32) | (unsigned)t));
    const float target = (float)(r >> 40) * (1.0f / 16777216.0f) * total;
    // the first class whose running sum exceeds the target (the last kept class when rounding leaves none)
    float run = incl - part;
    int pick = 0x7fffffff, last = -1;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        run += w[u];
        if (w[u] > 0.0f) {
            last = 4 * lane + u;
            if (run > target && pick == 0x7fffffff) pick = 4 * lane + u;
        }
    }
    // classes grow with the lane: the first lane with a pick holds the smallest, the last with a kept class the largest
    const unsigned long long pm = __ballot(pick != 0x7fffffff);
    if (pm) return __builtin_amdgcn_readlane(pick, __builtin_ctzll(pm));
    const unsigned long long lm = __ballot(last >= 0);
    return lm ? __builtin_amdgcn_readlane(last, 63 - __builtin_clzll(lm)) : -1;
}

// One round of the router descent from its ballot: node j of the round's subtree (breadth-first, j < 2^h - 1) goes
// right when bit 4 j of mask is set, and bits of nodes j >= 2^h - 1 are clear. Returns the node index reached after
// h <= 4 levels, in [2^h - 1, 2^(h+1) - 2]. The walk always takes 4 levels on l4 = 4 node (a bit test, a select and
// a shift-add in scalar registers per level); past level h it only goes left (clear bits), so
// loc_h + 1 = (loc_4 + 1) >> (4 - h).
__device__ __forceinline__ int walk_round(unsigned long long mask, int h) {
    unsigned l4 = 0, t;
    asm("s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 8, 4\n\t"
        "s_lshl1_add_u32 %0, %0, %1\n\t"
        "s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 8, 4\n\t"
        "s_lshl1_add_u32 %0, %0, %1\n\t"
        "s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 8, 4\n\t"
        "s_lshl1_add_u32 %0, %0, %1\n\t"
        "s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 8, 4\n\t"
        "s_lshl1_add_u32 %0, %0, %1"
        : "+s"(l4), "=&s"(t)
        : "s"(mask)
        : "scc");
    return (int)(((l4 >> 2) + 1) >> (4 - h)) - 1;
}

// walk_round for a ballot with node j's bit at bit j (one lane per node)
__device__ __forceinline__ int walk_bits(unsigned long long mask, int h) {
    unsigned l = 0, t;
    asm("s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 2, 1\n\t"
        "s_lshl1_add_u32 %0, %0, %1\n\t"
        "s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 2, 1\n\t"
        "s_lshl1_add_u32 %0, %0, %1\n\t"
        "s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 2, 1\n\t"
        "s_lshl1_add_u32 %0, %0, %1\n\t"
        "s_bitcmp1_b64 %2, %0\n\t"
        "s_cselect_b32 %1, 2, 1\n\t"
        "s_lshl1_add_u32 %0, %0, %1"
        : "+s"(l), "=&s"(t)
        : "s"(mask)
        : "scc");
    return (int)((l + 1) >> (4 - h)) - 1;
}

// the lanes whose pred holds, as a wavefront-uniform 64-bit mask
__device__ __forceinline__ unsigned long long lane_mask(bool pred) { return __builtin_amdgcn_ballot_w64(pred); }

// _mm512_cvtps_epi32 in round-to-nearest-even: NaN and |x| >= 2^31 give INT32_MIN (cpu/ygg.cpp:292 and others)
__device__ __forceinline__ int cvt_rne(float x) {
    return (x >= -2147483648.0f && x < 2147483648.0f) ? (int)__builtin_rintf(x) : (int)0x80000000;
}
__device__ __forceinline__ int clamp127(int v) { return v > 127 ? 127 : (v < -127 ? -127 : v); }
__device__ __forceinline__ int sat8(int v) { return v > 127 ? 127 : (v < -128 ? -128 : v); }
__device__ __forceinline__ int wadd(int a, int b) { return (int)((uint32_t)a + (uint32_t)b); }
__device__ __forceinline__ int sbyte(uint32_t w, int k) { return (int)(int8_t)(w >> (8 * k)); }
// two int8 (bytes k, k+1 of w) as an int16 pair
__device__ __forceinline__ uint32_t pair16(uint32_t w, int k) {
    return ((uint32_t)sbyte(w, k) & 0xFFFFu) | ((uint32_t)sbyte(w, k + 1) << 16);
}

// NW dwords from p, which is aligned to ALIGN bytes
template <int NW, int ALIGN>
__device__ __forceinline__ void load_words(uint32_t (&d)[NW], const void *p) {
    if constexpr (ALIGN % 16 == 0 && NW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 4; i++) {
            const uint4 v = ((const uint4 *)p)[i];
            d[4 * i] = v.x; d[4 * i + 1] = v.y; d[4 * i + 2] = v.z; d[4 * i + 3] = v.w;
        }
    } else if constexpr (ALIGN % 8 == 0 && NW % 2 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 2; i++) {
            const uint2 v = ((const uint2 *)p)[i];
            d[2 * i] = v.x; d[2 * i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NW; i++) d[i] = ((const uint32_t *)p)[i];
    }
}

// the same with non-temporal loads, for the per-expert streams that are read once per stream and token
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
template <int NW, int ALIGN>
__device__ __forceinline__ void load_words_nt(uint32_t (&d)[NW], const void *p) {
    if constexpr (ALIGN % 16 == 0 && NW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 4; i++) {
            const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p + i);
            d[4 * i] = v.x; d[4 * i + 1] = v.y; d[4 * i + 2] = v.z; d[4 * i + 3] = v.w;
        }
    } else if constexpr (ALIGN % 8 == 0 && NW % 2 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 2; i++) {
            const u32x2 v = __builtin_nontemporal_load((const u32x2 *)p + i);
            d[2 * i] = v.x; d[2 * i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NW; i++) d[i] = __builtin_nontemporal_load((const uint32_t *)p + i);
    }
}
__device__ __forceinline__ uint4 load16_nt(const void *p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// plain or non-temporal, chosen at compile time
template <bool NT> __device__ __forceinline__ uint4 load16(const void *p) {
    if constexpr (NT) return load16_nt(p);
    else return *(const uint4 *)p;
}
template <bool NT, int NW, int ALIGN> __device__ __forceinline__ void load_words_sel(uint32_t (&d)[NW], const void *p) {
    if constexpr (NT) load_words_nt<NW, ALIGN>(d, p);
    else load_words<NW, ALIGN>(d, p);
}
template <bool NT> __device__ __forceinline__ int load_i16(const int16_t *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

constexpr unsigned long long kDigestMul = 0x100000001B3ull;
constexpr unsigned long long kDigestLeaf = 0xD6E8FEB86659FD93ull;
constexpr unsigned long long kDigestCoord = 0x9E3779B97F4A7C15ull;

// GEN: sample the next input from the logits of every token (io.gen), instead of reading it from tokens
template <int N, int BLK, int R, bool GEN>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4))) void run_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int T,
                                                 int8_t *__restrict__ state, const YggIO io) {
    float *__restrict__ logits = io.logits;
    int32_t *__restrict__ leaves = io.leaves;
    int8_t *__restrict__ states = io.states;
    unsigned long long *__restrict__ digest = io.digest;
    const int32_t *__restrict__ targets = io.targets;
    double *__restrict__ nll = io.nll;
    constexpr int C = Lanes<N>::C, NL = Lanes<N>::NL;
    constexpr int Q4 = N / 4, QW = Q4 / 4;                       // quad-lane chunk of a row
    constexpr int QA = (Q4 % 16 == 0) ? 16 : 8;                  // its alignment
    constexpr int RL = ReadoutLanes<N, R>::RL, SP = ReadoutLanes<N, R>::SP, GP = ReadoutLanes<N, R>::GP;
    constexpr int SPW = SP / 4;
    constexpr int AW = C * BLK / 2;                              // A dwords per lane
    constexpr int NA = AW / 4;                                   // 16-byte A chunks per lane
    constexpr float kInvN = 1.0f / (float)N;

    __shared__ __attribute__((aligned(16))) int8_t qs[YGG_MAX_LAYERS * N];
    __shared__ __attribute__((aligned(16))) int8_t zls[YGG_MAX_RANK];
    __shared__ __attribute__((aligned(16))) int8_t zqs[32];

    const int lane = threadIdx.x;
    const int s = blockIdx.x;
    const int L = m.L, V = m.V, VP = m.VP, E = m.E, R2 = m.R2, K = m.K;
    const int qk = lane & 3, qj = lane >> 2;                     // quad lane, quad
    const int rj = lane / RL, rk = lane % RL;                    // readout row, readout lane

    int8_t *st = state + (size_t)s * L * N;
    for (int i = lane; i < L * N; i += 64) qs[i] = st[i];
    for (int i = lane; i < YGG_MAX_RANK; i += 64) zls[i] = 0;
    __syncthreads();
    unsigned long long dg = digest ? digest[s] : 0ull;
    NllSum nacc;
    const int32_t *tok = tokens + (size_t)s * (GEN ? 1 : T);
    int x_next = T > 0 ? __builtin_amdgcn_readfirstlane(tok[0]) : 0;

    for (int t = 0; t < T; t++) {
        const int x = x_next;
        if (!GEN && t + 1 < T) x_next = __builtin_amdgcn_readfirstlane(tok[t + 1]);
        if (x < 0 || x >= V) {
            if (lane == 0) atomicOr(m.err, 1u);
            break;
        }
        float lg[4];
#pragma unroll
        for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? m.output_bias[4 * lane + u] : 0.0f;

        for (int l = 0; l < L; l++) {
            const YggDevLayer &y = m.layers[l];
            int r = x;
            float rho = 0.0f;
            uint32_t qbw[QW];
            if (l > 0) {
                const int8_t *qb = qs + (l - 1) * N;
                load_words<QW, QA>(qbw, qb + qk * Q4);
                // rho: lane g < n/16 holds the sum of squares of coordinates [16 g, 16 g + 16)
                int sg = 0;
                if (lane < N / 16) {
                    uint32_t g4[4];
                    load_words<4, 16>(g4, qb + 16 * lane);
#pragma unroll
                    for (int i = 0; i < 4; i++) sg = dot4(g4[i], g4[i], sg);
                }
                if (y.r2b) {
                    float sum = 0.0f;
#pragma unroll
                    for (int g = 0; g < N / 16; g++) sum = sum + y.r2b[g] * (float)__builtin_amdgcn_readlane(sg, g);
                    rho = 1.0f / sqrtf(sum * kInvN + y.rms_eps);
                } else {
                    int S = 0;
#pragma unroll
                    for (int g = 0; g < N / 16; g++) S += __builtin_amdgcn_readlane(sg, g);
                    rho = 1.0f / sqrtf((float)S * kInvN + y.rms_eps);
                }
                // router descent, up to 4 levels per round
                const float *thr = y.thr + (size_t)x * y.thr_stride;
                int ix = 1, base = 0, d0 = 0;
                for (int rd = 0; rd < m.n_rounds; rd++) {
                    const int h = m.round_h[rd];
                    const int nn = (1 << h) - 1;
                    const int slot = base + ((ix - (1 << d0)) << h) + qj;
                    int dot = 0;
                    float th = 0.0f;
                    if (qj < nn) {
                        uint32_t wv[QW];
                        load_words<QW, QA>(wv, y.w + (size_t)slot * N + qk * Q4);
                        th = thr[slot];
#pragma unroll
                        for (int i = 0; i < QW; i++) dot = dot4(wv[i], qbw[i], dot);
                    }
                    dot = sum4(dot);
                    const bool right = (float)dot * rho > th;
                    const int loc = walk_round(lane_mask(right && qk == 0 && qj < nn), h);
                    base += (1 << d0) << h;
                    d0 += h;
                    ix = (ix << h) + (loc - nn);
                }
                r = ix - E;
            }

            // the expert's gather record and table row
            const uint8_t *g = y.gath + (size_t)r * y.gath_bytes;
            uint32_t aw[AW];
            uint32_t pw[SPW];
            int trow[C];
            if (lane < NL) {
#pragma unroll
                for (int c = 0; c < NA; c++) {
                    const uint4 v = *(const uint4 *)(g + (c * NL + lane) * 16);
                    aw[4 * c] = v.x; aw[4 * c + 1] = v.y; aw[4 * c + 2] = v.z; aw[4 * c + 3] = v.w;
                }
                if (y.table) {
                    const int16_t *tr = y.table + (size_t)r * y.table_sr + (size_t)x * y.table_sx + C * lane;
#pragma unroll
                    for (int c = 0; c < C; c++) trow[c] = tr[c];
                }
            }
            {
                const uint8_t *pp = g + y.off_P;
#pragma unroll
                for (int gi = 0; gi < SP / GP; gi++) {
                    uint32_t tmp[GP / 4];
                    load_words<GP / 4, GP>(tmp, pp + (gi * 64 + lane) * GP);
#pragma unroll
                    for (int i = 0; i < GP / 4; i++) pw[gi * (GP / 4) + i] = tmp[i];
                }
            }

            // layer input zl from V' (cpu/ygg.cpp:285-296)
            if (l > 0 && R2 > 0) {
                const int RG = (R2 + 15) >> 4;
                // (unrolled: the row loads of several passes are in flight together)
#pragma unroll 4
                for (int gg = 0; gg < RG; gg++) {
                    const int k = gg * 16 + qj;
                    uint32_t vv[QW];
                    load_words<QW, QA>(vv, y.vl + (size_t)k * N + qk * Q4);
                    int a = 0;
#pragma unroll
                    for (int i = 0; i < QW; i++) a = dot4(vv[i], qbw[i], a);
                    a = sum4(a);
                    if (qk == 0) {
                        float zf = (float)a * y.mv[k];
                        zf = zf * rho;
                        zls[k] = (int8_t)clamp127(cvt_rne(zf));
                    }
                }
            }
            __syncthreads();

            // transition + input + layer input -> sat8 (cpu/ygg.cpp:311-389)
            int qn[C];
            if (lane < NL) {
                const int blk0 = (C * lane / BLK) * BLK;
                uint32_t qv[BLK / 4];
                load_words<BLK / 4, BLK>(qv, qs + l * N + blk0);
                uint32_t qp[BLK / 2];
#pragma unroll
                for (int i = 0; i < BLK / 4; i++) { qp[2 * i] = pair16(qv[i], 0); qp[2 * i + 1] = pair16(qv[i], 2); }
                int acc[C];
#pragma unroll
                for (int c = 0; c < C; c++) {
                    int a = 0;
#pragma unroll
                    for (int p = 0; p < BLK / 2; p++) a = dot2(aw[c * (BLK / 2) + p], qp[p], a);
                    acc[c] = (a + (1 << (m.shift - 1))) >> m.shift;
                }
                if (y.table) {
#pragma unroll
                    for (int c = 0; c < C; c++) acc[c] = wadd(acc[c], trow[c]);
                } else {
                    // factored: rint(f32(U_r v[x]) * f32(su_r * mT_i)) + c_r (cpu/ygg.cpp:339-358)
                    const uint8_t *fp = g + y.off_F;
                    const uint32_t *vx = (const uint32_t *)(y.vt + (size_t)x * K);
                    int d[C];
#pragma unroll
                    for (int c = 0; c < C; c++) d[c] = 0;
#pragma unroll 8
                    for (int k4 = 0; k4 < K / 4; k4++) {
                        const uint32_t vw = vx[k4];
                        const uint32_t *up = (const uint32_t *)(fp + ((size_t)(k4 * NL + lane) * C) * 4);
#pragma unroll
                        for (int c = 0; c < C; c++) d[c] = dot4(up[c], vw, d[c]);
                    }
                    const float su = *(const float *)(g + y.off_FS);
                    const int16_t *cb = (const int16_t *)(g + y.off_FB) + C * lane;
#pragma unroll
                    for (int c = 0; c < C; c++) {
                        const float mul = su * y.mT[C * lane + c];
                        acc[c] = wadd(acc[c], wadd(cvt_rne((float)d[c] * mul), cb[c]));
                    }
                }
                if (l > 0 && R2 > 0) {
                    // rint(f32(U'_r zl) * m_ul) (cpu/ygg.cpp:360-377)
                    const uint8_t *up0 = g + y.off_U;
                    int d[C];
#pragma unroll
                    for (int c = 0; c < C; c++) d[c] = 0;
#pragma unroll 8
                    for (int k4 = 0; k4 < R2 / 4; k4++) {
                        const uint32_t zw = ((const uint32_t *)zls)[k4];
                        const uint32_t *up = (const uint32_t *)(up0 + ((size_t)(k4 * NL + lane) * C) * 4);
#pragma unroll
                        for (int c = 0; c < C; c++) d[c] = dot4(up[c], zw, d[c]);
                    }
#pragma unroll
                    for (int c = 0; c < C; c++) {
                        const float mu = y.mulv ? y.mulv[C * lane + c] : y.layer_input_scale;
                        acc[c] = wadd(acc[c], cvt_rne((float)d[c] * mu));
                    }
                }
#pragma unroll
                for (int c = 0; c < C; c++) qn[c] = sat8(acc[c]);
            }
            __syncthreads();
            if (lane < NL) {
#pragma unroll
                for (int c = 0; c < C; c++) qs[l * N + C * lane + c] = (int8_t)qn[c];
            }
            __syncthreads();

            // readout zq = sat(rint(f32(P_r q) m_z)) and the unembedding (cpu/ygg.cpp:395-435)
            {
                uint32_t qv[SPW];
                load_words<SPW, (SP % 16 == 0 ? 16 : (SP % 8 == 0 ? 8 : 4))>(qv, qs + l * N + rk * SP);
                int z = 0;
#pragma unroll
                for (int i = 0; i < SPW; i++) z = dot4(pw[i], qv[i], z);
                z = group_sum<RL>(z);
                if (rk == 0) {
                    const float mz = y.mz ? y.mz[(size_t)r * R + rj] : y.readout_scale;
                    zqs[rj] = (int8_t)clamp127(cvt_rne((float)z * mz));
                }
            }
            __syncthreads();
            if (4 * lane < VP) {
                uint32_t zw[R / 4];
                load_words<R / 4, 16>(zw, zqs);
                const int8_t *Qr = y.Q + (size_t)(4 * lane) * R;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    uint32_t qq[R / 4];
                    load_words<R / 4, 8>(qq, Qr + u * R);
                    int d = 0;
#pragma unroll
                    for (int i = 0; i < R / 4; i++) d = dot4(qq[i], zw[i], d);
                    const float sc = y.sqv ? y.sqv[4 * lane + u] : y.unembed_scale;
                    lg[u] = lg[u] + (float)d * sc;
                }
            }
            if (leaves && lane == 0) leaves[((size_t)s * T + t) * L + l] = r;
            if (digest) {
                unsigned long long f = 0;
                if (lane < NL) {
#pragma unroll
                    for (int c = 0; c < C; c++)
                        f += (unsigned long long)((uint8_t)qn[c] + 1u) *
                             ((unsigned long long)(2 * (C * lane + c) + 1) * kDigestCoord);
                }
                f = wave_sum_u64(f);
                dg = dg * kDigestMul + ((unsigned long long)(uint32_t)r * kDigestLeaf + f + (unsigned long long)l);
            }
            __syncthreads();
        }

        if (logits) {
            float *o = logits + ((size_t)s * T + t) * V;
            if ((V & 3) == 0 && 4 * lane + 3 < V) {
                *(float4 *)(o + 4 * lane) = make_float4(lg[0], lg[1], lg[2], lg[3]);
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (4 * lane + u < V) o[4 * lane + u] = lg[u];
            }
        }
        if (nll) {
            const int yv = targets[(size_t)s * T + t];
            if (yv >= 0 && yv < V) token_nll(nacc, lg, V, yv, lane);
            else if (lane == 0) atomicOr(m.err, 2u);
        }
        if (GEN) {
            x_next = __builtin_amdgcn_readfirstlane(sample_token(lg, V, io.temperature, io.top_k, io.seed, s, t, lane));
            if (lane == 0) io.gen[(size_t)s * T + t] = x_next;
        }
        if (states) {
            int8_t *so = states + ((size_t)s * T + t) * L * N;
            for (int i = lane; i < L * N; i += 64) so[i] = qs[i];
        }
    }
    __syncthreads();
    for (int i = lane; i < L * N; i += 64) st[i] = qs[i];
    if (digest && lane == 0) digest[s] = dg;
    if (nll && lane == 0) nll[s] += nacc.value();
}

}  // namespace ygg
