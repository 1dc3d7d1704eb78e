// Two kernels for the common shape: readout rank 8, block 16, layer-input rank 16, table storage, one scale per
// tensor, at most 4 layers (every benchmark configuration). Same arithmetic and lane mapping as run_kernel
// (ygg_kernel.h); the per-layer pieces below are shared by both.
//
// fast_kernel (throughput: many streams): one wavefront per stream runs every layer of every token, 4 streams per
// workgroup. Its DEEP form (generation for few streams: one stream per workgroup) shortens the router descent, see
// descend_deep. What every stream reads at every token is in LDS once per workgroup: the unembedding Q of every layer,
// the layer-input down-projection V' of every routed layer and the router rows of the first descent round (nodes
// 1..15). The thresholds of that round, thr[x][1..15], depend only on the token and are loaded when the token is
// read. An expert's whole gather record (A16, U', P) and table row are loaded in one burst as soon as the expert is
// known (plain loads: non-temporal ones cut the fetched bytes by 6% but made the step 36% slower). LDS exchanges
// inside a wavefront are ordered by wave-level fences, so the streams of a workgroup never wait for each other.
//
// pipe_kernel (latency: few streams): one workgroup per stream and one wavefront per layer. In tick k wavefront l
// processes token k - l, so the L layers of a stream work on L consecutive tokens at once and a token costs about
// one layer's chain of dependent loads instead of L of them. Layer l at token t needs the state of layer l - 1 at
// token t (written by wavefront l - 1 in tick k - 1) and its own state at token t - 1 (double-buffered by token
// parity); one workgroup barrier per tick orders them. Logits of a token are summed layer by layer in a ring of L
// LDS rows in layer order (as the reference does, cpu/ygg.cpp:457) and stored by the last layer's wavefront. The
// token layer's gather record and the routed layers' first-round thresholds of the next token are loaded a tick
// ahead.
#pragma once
#include <type_traits>

#include "ygg_kernel.h"

namespace ygg {

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kFastWaves = 4;

// constants of a state width N (block 16)
template <int N> struct Fast {
    static constexpr int BLK = 16;
    static constexpr int C = Lanes<N>::C, NL = Lanes<N>::NL;
    static constexpr int Q4 = N / 4, QW = Q4 / 4;
    static constexpr int QA = (Q4 % 16 == 0) ? 16 : 8;
    static constexpr int AW = C * BLK / 2, NA = AW / 4;
    static constexpr float kInvN = 1.0f / (float)N;
};

// a specialised shape: state width N, readout rank R, layer-input rank R2 (a multiple of 4, 0: no layer input),
// transition block BLK (16 or 8)
template <int N_, int R_, int R2_, int BLK_ = 16> struct Shape : Fast<N_> {
    static constexpr int N = N_, R = R_, R2 = R2_, BLK = BLK_;
    static constexpr int AW = Fast<N_>::C * BLK / 2, NA = AW / 4;   // A hi/lo dwords and 16-byte chunks per lane
    static constexpr int RL = ReadoutLanes<N, R>::RL, SP = ReadoutLanes<N, R>::SP, GP = ReadoutLanes<N, R>::GP;
    static constexpr int SPW = SP / 4;
    static constexpr int SPA = SP % 16 == 0 ? 16 : (SP % 8 == 0 ? 8 : 4);
    static constexpr int K4 = R2 / 4;      // U' dwords per coordinate
    static constexpr int K4A = K4 > 0 ? K4 : 1;                     // (array extent)
    static constexpr int RG = (R2 + 15) / 16;      // passes of 16 V' rows (V' is held zero-padded to 16 RG rows)
    static constexpr int R2P = 16 * RG, R2A = R2P > 0 ? R2P : 1;   // V' rows and m_v entries held; array extent
    static constexpr int QC = R / 4;       // 16-byte chunks of a lane's 4 unembedding classes
    static constexpr int ZQ = R > 16 ? R : 16, ZL = R2P > 16 ? R2P : 16;    // LDS bytes of zq and zl
};

// factored input storage (cpu/ygg.cpp:339-358): input ranks up to 64, this many dwords per coordinate
constexpr int kFactK4 = YGG_MAX_FACT_RANK / 4;

// the per-expert registers of one stream and layer. FACT: the model stores its routed inputs factored (the routed
// layers' records hold U_r, c_r and su_r instead of a table)
template <class SH, bool FACT = false> struct Gather {
    uint32_t aw[SH::AW], pw[SH::SPW], uw[SH::K4A][SH::C];
    // the table row's C int16 entries of this lane as loaded: packed in pairs (C >= 2) or one sign-extended entry
    // (C = 1); unpacked where the update reads them, so that nothing waits for the load in between. FACT, routed: the
    // factored bias c_r's entries, packed the same way
    int trw[(SH::C + 1) / 2];
    float mzr;             // group scales: the readout scale of this lane's readout row (m_z of the expert's row)
    uint32_t fw[FACT ? kFactK4 : 1][SH::C];   // FACT: U_r, this lane's C dwords per 4 ranks (the U' layout)
    float fs;                                  // FACT: su_r
};
template <class SH, bool FACT> __device__ __forceinline__ int table_entry(const Gather<SH, FACT> &G, int c) {
    if constexpr (SH::C == 1) return G.trw[0];
    else return (c & 1) ? (G.trw[c >> 1] >> 16) : (int)(int16_t)(G.trw[c >> 1] & 0xffff);
}

// A quad lane's share of an n-byte row: for n = 128 the 16-byte chunks at qk 16 and 64 + qk 16, with LDS rows
// kLdsRow = 192 bytes apart, so that the 16 quads of a wavefront reading 16 rows hit 64 distinct banks (contiguous
// 32-byte quarters of 128-byte rows put rows j and j + 2 on the same banks); otherwise the contiguous quarter qk Q4
// (n = 256: LDS rows 272 bytes apart, so that 4 consecutive rows start on 4 different 16-byte bank groups).
template <int N> constexpr int kLdsRow = N == 128 ? 192 : (N == 256 ? 272 : N);

template <int N>
__device__ __forceinline__ void quad_share(uint32_t (&w)[Fast<N>::QW], const int8_t *row, int qk) {
    using F = Fast<N>;
    if constexpr (N == 128) {
        uint32_t a[4], b[4];
        load_words<4, 16>(a, row + qk * 16);
        load_words<4, 16>(b, row + 64 + qk * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w[i] = a[i];
            w[4 + i] = b[i];
        }
    } else {
        load_words<F::QW, F::QA>(w, row + qk * F::Q4);
    }
}

// the workgroup's LDS copies of Q (all layers), V' and the first-round router rows (routed layers). Q is held in
// R / 4 planes of 1 KiB: the 4 R bytes of lane l's classes 4l .. 4l + 3 (class-major) as 16-byte chunks, chunk p at
// 16 l in plane p (R = 8: classes 4l, 4l + 1 in plane 0, 4l + 2, 4l + 3 in plane 1).
// WITHV = false: V' stays out of LDS (its user keeps the rows in registers)
template <class SH, int L, bool WITHV = true> struct SharedTables {
    static constexpr int LR = L > 1 ? L - 1 : 1;
    int8_t Q[L][256 * SH::R];
    int8_t W[LR][15 * kLdsRow<SH::N>];
    int8_t V[WITHV ? LR : 1][WITHV ? SH::R2A * kLdsRow<SH::N> : 16];
    float mv[LR][SH::R2A];
};

template <class SH, int L> constexpr int kTablesBytes = (int)sizeof(SharedTables<SH, L>);

// Models with group scales (cpu/ygg.cpp:257-266, 371-372, 398, 431): per layer the unembedding scale of every class
// (sqv, or the layer's single scale), per routed layer the layer-input scale of every coordinate (mulv, or the single
// scale) and the squared group scales of the layer below (r2b); the readout row scales (m_z per expert and row) come
// with the gather record.
template <class SH, int L> struct GroupTables {
    static constexpr int LR = L > 1 ? L - 1 : 1;
    float sq[L][256];
    float mul[LR][SH::N];
    float r2[LR][SH::N / 16];
};

struct NoGroupTables {
    int unused;
};
template <class SH, int L, bool GROUP>
using GroupTablesOf = std::conditional_t<GROUP, GroupTables<SH, L>, NoGroupTables>;

template <class SH, int L, int NT>
__device__ __forceinline__ void load_group_tables(GroupTables<SH, L> &G, const YggDevModel &m, int tid) {
    constexpr int N = SH::N, LR = L > 1 ? L - 1 : 1;
    constexpr int SK = (256 + NT - 1) / NT, MK = (N + NT - 1) / NT;
    float sv[L][SK], mv[LR][MK], rv = 0.0f;
#pragma unroll
    for (int l = 0; l < L; l++) {
        const YggDevLayer &y = m.layers[l];
#pragma unroll
        for (int k = 0; k < SK; k++) {
            const int c = tid + k * NT;
            sv[l][k] = y.unembed_scale;
            if (y.sqv && c < m.VP) sv[l][k] = y.sqv[c];
        }
    }
#pragma unroll
    for (int l = 1; l < L; l++) {
        const YggDevLayer &y = m.layers[l];
#pragma unroll
        for (int k = 0; k < MK; k++) {
            const int c = tid + k * NT;
            mv[l - 1][k] = y.layer_input_scale;
            if (y.mulv && c < N) mv[l - 1][k] = y.mulv[c];
        }
        if (y.r2b && tid / (N / 16) == l - 1) rv = y.r2b[tid % (N / 16)];
    }
#pragma unroll
    for (int l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < SK; k++)
            if (tid + k * NT < 256) G.sq[l][tid + k * NT] = sv[l][k];
#pragma unroll
    for (int l = 1; l < L; l++)
#pragma unroll
        for (int k = 0; k < MK; k++)
            if (tid + k * NT < N) G.mul[l - 1][tid + k * NT] = mv[l - 1][k];
    if (L > 1 && tid < (N / 16) * (L - 1)) G.r2[tid / (N / 16)][tid % (N / 16)] = rv;
}

// Stage the tables with NT threads: every load is issued before the first LDS store, so a launch waits for them
// once (a load-store loop would wait for each in turn).
template <class SH, int L, int NT, bool WITHV = true>
__device__ __forceinline__ void load_tables(SharedTables<SH, L, WITHV> &S, const YggDevModel &m, int tid) {
    // 16-byte chunks: RC per row in memory, SC per row in LDS
    constexpr int N = SH::N, R2 = SH::R2P, QC = SH::QC;      // (V' and m_v as held: R2 rounded up to 16)
    constexpr int RC = N / 16, SC = kLdsRow<N> / 16, LR = L > 1 ? L - 1 : 1;
    constexpr int QK = (16 * SH::R + NT - 1) / NT;     // Q chunks (at most 16 R: VP <= 256) per thread and layer
    constexpr int VR = 15 + (WITHV ? R2 : 0);          // first-round rows and V' rows of a routed layer
    constexpr int RK = (VR * RC + NT - 1) / NT;        // their chunks per thread
    constexpr int R2D = R2 > 0 ? R2 : 1, MVN = L > 1 ? R2 * (L - 1) : 0;   // m_v entries: MVK per thread
    constexpr int MVK = MVN > 0 ? (MVN + NT - 1) / NT : 1;
    const int qch = m.VP * SH::R / 16, rows = (1 << m.round_h[0]) - 1;
    uint4 qv[L][QK], rv[LR][RK];
    float mvv[MVK];
#pragma unroll
    for (int l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < QK; k++) {
            const int c = tid + k * NT;
            qv[l][k] = make_uint4(0u, 0u, 0u, 0u);
            if (c < qch) qv[l][k] = ((const uint4 *)m.layers[l].Q)[c];
        }
#pragma unroll
    for (int l = 1; l < L; l++) {
        const YggDevLayer &y = m.layers[l];
#pragma unroll
        for (int k = 0; k < RK; k++) {
            const int c = tid + k * NT;
            rv[l - 1][k] = make_uint4(0u, 0u, 0u, 0u);
            if (c < rows * RC)
                rv[l - 1][k] = ((const uint4 *)y.w)[c];
            else if (c >= 15 * RC && c < VR * RC)
                rv[l - 1][k] = ((const uint4 *)y.vl)[c - 15 * RC];
        }
    }
#pragma unroll
    for (int k = 0; k < MVK; k++) {
        const int c = tid + k * NT;
        mvv[k] = 0.0f;
#pragma unroll
        for (int l = 1; l < L; l++)
            if (c < MVN && c / R2D == l - 1) mvv[k] = m.layers[l].mv[c % R2D];
    }
#pragma unroll
    for (int l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < QK; k++) {
            const int c = tid + k * NT;
            if (c < qch) ((uint4 *)S.Q[l])[(c % QC) * 64 + c / QC] = qv[l][k];
        }
#pragma unroll
    for (int l = 1; l < L; l++)
#pragma unroll
        for (int k = 0; k < RK; k++) {
            const int c = tid + k * NT;
            if (c < 15 * RC)
                ((uint4 *)S.W[l - 1])[(c / RC) * SC + c % RC] = rv[l - 1][k];
            else if (WITHV && c < VR * RC)
                ((uint4 *)S.V[l - 1])[((c - 15 * RC) / RC) * SC + (c - 15 * RC) % RC] = rv[l - 1][k];
        }
#pragma unroll
    for (int k = 0; k < MVK; k++)
        if (tid + k * NT < MVN) S.mv[(tid + k * NT) / R2D][(tid + k * NT) % R2D] = mvv[k];
}

// load_tables for the one-token build, in layer order. Unit j is layer j's unembedding Q and, for a routed layer
// (j >= 1), its first-round rows and V' rows (unit 0 also carries every m_v). Every load is issued first, in unit
// order, then each unit's stores, after which the wavefront adds 1 to *done (LDS, workgroup scope): unit j is in LDS
// once *done reaches NW (j + 1), NW the staging wavefronts. The stream's wavefront waits for a routed layer's unit
// before that layer's descent instead of for every table at once (the widest shape stages 129 KB).
template <class SH, int L, int NT>
__device__ __forceinline__ void load_tables_units(SharedTables<SH, L, true> &S, const YggDevModel &m, int tid,
                                                  uint32_t *done) {
    constexpr int N = SH::N, R2 = SH::R2P, QC = SH::QC;
    constexpr int RC = N / 16, SC = kLdsRow<N> / 16, LR = L > 1 ? L - 1 : 1;
    constexpr int QK = (16 * SH::R + NT - 1) / NT;
    constexpr int VR = 15 + R2;
    constexpr int RK = (VR * RC + NT - 1) / NT;
    constexpr int R2D = R2 > 0 ? R2 : 1, MVN = L > 1 ? R2 * (L - 1) : 0;
    constexpr int MVK = MVN > 0 ? (MVN + NT - 1) / NT : 1;
    const int qch = m.VP * SH::R / 16, rows = (1 << m.round_h[0]) - 1;
    uint4 qv[L][QK], rv[LR][RK];
    float mvv[MVK];
#pragma unroll
    for (int k = 0; k < MVK; k++) {
        const int c = tid + k * NT;
        mvv[k] = 0.0f;
#pragma unroll
        for (int l = 1; l < L; l++)
            if (c < MVN && c / R2D == l - 1) mvv[k] = m.layers[l].mv[c % R2D];
    }
#pragma unroll
    for (int j = 0; j < L; j++) {
#pragma unroll
        for (int k = 0; k < QK; k++) {
            const int c = tid + k * NT;
            qv[j][k] = make_uint4(0u, 0u, 0u, 0u);
            if (c < qch) qv[j][k] = ((const uint4 *)m.layers[j].Q)[c];
        }
        if (j >= 1) {
            const YggDevLayer &y = m.layers[j];
#pragma unroll
            for (int k = 0; k < RK; k++) {
                const int c = tid + k * NT;
                rv[j - 1][k] = make_uint4(0u, 0u, 0u, 0u);
                if (c < rows * RC)
                    rv[j - 1][k] = ((const uint4 *)y.w)[c];
                else if (c >= 15 * RC && c < VR * RC)
                    rv[j - 1][k] = ((const uint4 *)y.vl)[c - 15 * RC];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < L; j++) {
        if (j == 0) {
#pragma unroll
            for (int k = 0; k < MVK; k++)
                if (tid + k * NT < MVN) S.mv[(tid + k * NT) / R2D][(tid + k * NT) % R2D] = mvv[k];
        }
#pragma unroll
        for (int k = 0; k < QK; k++) {
            const int c = tid + k * NT;
            if (c < qch) ((uint4 *)S.Q[j])[(c % QC) * 64 + c / QC] = qv[j][k];
        }
        if (j >= 1) {
#pragma unroll
            for (int k = 0; k < RK; k++) {
                const int c = tid + k * NT;
                if (c < 15 * RC)
                    ((uint4 *)S.W[j - 1])[(c / RC) * SC + c % RC] = rv[j - 1][k];
                else if (c < VR * RC)
                    ((uint4 *)S.V[j - 1])[((c - 15 * RC) / RC) * SC + (c - 15 * RC) % RC] = rv[j - 1][k];
            }
        }
        // (the wavefront's LDS stores done, then its count; the wavefront runs in lockstep)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if ((tid & 63) == 0) __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// the stream's wait for *done >= need (load_tables_units); the staging wavefronts wait on nothing, so the count
// arrives; the wall-clock bound (1 ms, then error bit 4) only keeps a fault elsewhere from becoming a hang
__device__ __forceinline__ void stage_wait(const uint32_t *done, uint32_t need, uint32_t *err, int lane) {
    const uint64_t t0 = wall_clock64();
    while (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < need) {
        __builtin_amdgcn_s_sleep(1);
        if (wall_clock64() - t0 > 100000) {
            if (lane == 0) atomicOr(err, 4u);
            break;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Touch every 64-byte line of the kernel argument (the model description, read by scalar loads) at entry: the
// scalar cache starts each launch cold, and a layer's fields would otherwise first be read when that layer starts
// (worth 1 us in a launch of one token; launches of many tokens do without).
// The fields touched lie less than 64 bytes apart and are ones the token loop never reads (format variants, LDS
// staging sources), so the compiler has nothing to keep live from here on.
template <int L>
__device__ __forceinline__ void touch_args(const YggDevModel &m) {
    asm volatile("; args %0 %1" ::"s"(m.BLK), "s"(m.round_h[12]));
#pragma unroll
    for (int l = 0; l < L; l++)
        asm volatile("; layer args %0 %1 %2 %3 %4" ::"s"(m.layers[l].vl), "s"(m.layers[l].r2b), "s"(m.layers[l].vt),
                     "s"(m.layers[l].mT), "s"(m.layers[l].off_FS));
}

// the quad-lane chunk of the state below and rho = 1 / sqrt(mean(q^2) + eps) (cpu/ygg.cpp:248-255)
template <int N>
__device__ __forceinline__ float below_and_rho(uint32_t (&qbw)[Fast<N>::QW], const int8_t *qb, float eps, int lane) {
    using F = Fast<N>;
    quad_share<N>(qbw, qb, lane & 3);
    // the 4 lanes of every quad hold the whole state between them: exact sum of squares by a quad sum
    int S = 0;
#pragma unroll
    for (int i = 0; i < F::QW; i++) S = dot4(qbw[i], qbw[i], S);
    S = sum4(S);
    return 1.0f / sqrtf((float)S * F::kInvN + eps);
}

// rho with group scales: sum over the 16-coordinate groups g, in order, of r2b[g] f32(sum of q^2 over g), then
// 1 / sqrt(sum / n + eps) (cpu/ygg.cpp:257-266). r2 the layer's r2b (LDS); qbw the quad share as below_and_rho loads
// it: quad lane k holds group k (n = 64), groups k and 4 + k (n = 128) or groups 4k .. 4k + 3 (n = 256).
template <int N>
__device__ __forceinline__ float group_rho(const uint32_t (&qbw)[Fast<N>::QW], const float *r2, float eps) {
    static_assert(N == 64 || N == 128 || N == 256, "groups whole in a quad lane's share");
    constexpr int GPL = Fast<N>::QW / 4;        // groups per quad lane
    int sg[GPL];
#pragma unroll
    for (int j = 0; j < GPL; j++) {
        sg[j] = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) sg[j] = dot4(qbw[4 * j + i], qbw[4 * j + i], sg[j]);
    }
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < N / 16; g++) {
        // the lane and slot of group g
        const int ln = N == 128 ? (g & 3) : (N == 256 ? g >> 2 : g);
        const int j = N == 128 ? (g >> 2) : (N == 256 ? (g & 3) : 0);
        sum = sum + r2[g] * (float)__builtin_amdgcn_readlane(sg[j], ln);
    }
    return 1.0f / sqrtf(sum * Fast<N>::kInvN + eps);
}

// nothing to overlap with the first global router round
struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

// the router descent (cpu/ygg.cpp:271-280) -> leaf index; the first round from the LDS rows W0 and the thresholds
// th0 (thr[x][slot qj] of that round, loaded by the caller), the others from global memory. hook() runs once, while
// the loads of the first global round are in flight (or after the descent when there is no such round).
template <int N, class Hook = NoHook>
__device__ __forceinline__ int descend(const YggDevModel &m, const YggDevLayer &y, const int8_t *W0, float th0,
                                       const uint32_t (&qbw)[Fast<N>::QW], float rho, int x, int lane,
                                       Hook hook = Hook()) {
    using F = Fast<N>;
    const int qk = lane & 3, qj = lane >> 2;
    const int h1 = m.round_h[0], nn1 = (1 << h1) - 1;
    int ix;
    {
        int dot = 0;
        if (qj < nn1) {
            uint32_t wv[F::QW];
            quad_share<N>(wv, W0 + qj * kLdsRow<N>, qk);
#pragma unroll
            for (int i = 0; i < F::QW; i++) dot = dot4(wv[i], qbw[i], dot);
        }
        dot = sum4(dot);
        const bool right = (float)dot * rho > th0;
        const int loc = walk_round(lane_mask(right && qk == 0 && qj < nn1), h1);
        ix = (1 << h1) + (loc - nn1);
    }
    const float *thr = y.thr + (size_t)x * y.thr_stride;
    int base = 1 << h1, d0 = h1;
    for (int rd = 1; rd < m.n_rounds; rd++) {
        const int h = (m.round_pack >> (4 * rd)) & 15;
        const int nn = (1 << h) - 1;
        const int blk = base + ((ix - (1 << d0)) << h);
        // only the quads of the round's nodes load (a quad past them would fetch another cache line)
        const int slot = blk + qj;
        uint32_t wv[F::QW];
        float th = 0.0f;
        if (qj < nn) {
            quad_share<N>(wv, y.w + (size_t)slot * N, qk);
            th = thr[slot];
        }
        if (rd == 1) hook();
        int dot = 0;
        if (qj < nn) {
#pragma unroll
            for (int i = 0; i < F::QW; i++) dot = dot4(wv[i], qbw[i], dot);
        }
        dot = sum4(dot);
        const bool right = (float)dot * rho > th;
        const int loc = walk_round(lane_mask(right && qk == 0 && qj < nn), h);
        base += (1 << d0) << h;
        d0 += h;
        ix = (ix << h) + (loc - nn);
    }
    if (m.n_rounds == 1) hook();
    return ix - m.E;
}

// ------------------------------------------------------------------------------------------ deep descent
// For one stream generating tokens, every router round is a dependent step on the path from one sampled token to the
// next. The deep descent takes the second round from LDS (its rows staged once per launch, its thresholds loaded
// with the token) and evaluates the rounds after it (at most two, at most 6 levels together) as one round, so a
// routed layer's descent has a single dependent global round. It needs a plan of 2 to 4 rounds whose first has at
// least 2 levels (16-byte aligned threshold blocks).

// The second round's rows of one routed layer in LDS: slot s of the round (s < 2^(h0 + h1) <= 256) at s N. For
// n = 128 the two 64-byte halves of a row are swapped when bit 1 of s is set: the 16 quads of a wavefront reading
// 16 consecutive rows then hit 64 distinct banks in every 16-lane group.
template <int N> constexpr int kR2Slots = 256;

template <int N, int L, int NT>
__device__ __forceinline__ void load_round2(int8_t (*W1)[kR2Slots<N> * N], const YggDevModel &m, int tid) {
    constexpr int RC = N / 16, K = (kR2Slots<N> * RC + NT - 1) / NT, LR = L > 1 ? L - 1 : 1;
    if (m.n_rounds < 2) return;
    const int base = 1 << m.round_h[0], count = (1 << (m.round_h[0] + m.round_h[1])) * RC;
    // every load first, then the stores
    uint4 v[LR][K];
#pragma unroll
    for (int l = 1; l < L; l++) {
        const uint4 *src = (const uint4 *)(m.layers[l].w + (size_t)base * N);
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int c = tid + k * NT;
            v[l - 1][k] = make_uint4(0u, 0u, 0u, 0u);
            if (c < count) v[l - 1][k] = src[c];
        }
    }
#pragma unroll
    for (int l = 1; l < L; l++)
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int c = tid + k * NT, sl = c / RC, q = c % RC;
            if (c < count) ((uint4 *)W1[l - 1])[sl * RC + (N == 128 ? q ^ (((sl >> 1) & 1) << 2) : q)] = v[l - 1][k];
        }
}

// quad_share of slot sl of the LDS second-round rows
template <int N>
__device__ __forceinline__ void quad_share_r2(uint32_t (&w)[Fast<N>::QW], const int8_t *row, int qk, int sl) {
    if constexpr (N == 128) {
        const int sw = ((sl >> 1) & 1) * 64;
        uint32_t a[4], b[4];
        load_words<4, 16>(a, row + qk * 16 + sw);
        load_words<4, 16>(b, row + qk * 16 + (64 - sw));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w[i] = a[i];
            w[4 + i] = b[i];
        }
    } else {
        quad_share<N>(w, row, qk);
    }
}

// The tail round: the rounds after the second as one round with one lane per node (at most 63): lanes
// [0, 2^h2 - 1) take the third round's block (breadth-first), the next 2^h2 (2^h3 - 1) lanes the 2^h2 fourth-round
// blocks below it, which lie one after the other; other lanes are off. Lane l's node sits in slot ta + (sub << tsh),
// sub the index of the second round's end node among the nodes of its depth d2 = h0 + h1. Each lane reads its whole
// row and forms the dot alone (measured faster here than quads over several passes, whose reductions and shuffles
// lengthen the chain).
struct Tail {
    int ta, tsh;
    bool on;
};

// (r0 = 1, the one-token build's folded tail: the second and third rounds of a three-round plan)
__device__ __forceinline__ Tail make_tail(const YggDevModel &m, int lane, int r0 = 2) {
    Tail t{0, 0, false};
    if (m.n_rounds < r0 + 1) return t;
    const int h0 = m.round_h[0], hb = r0 == 2 ? m.round_h[1] : 0;       // the levels before the tail: h0 + hb
    const int h2 = m.round_h[r0], h3 = m.n_rounds > r0 + 1 ? m.round_h[r0 + 1] : 0;
    const int base2 = (1 << h0) + (r0 == 2 ? 1 << (h0 + hb) : 0), base3 = base2 + (1 << (h0 + hb + h2));
    const int nn2 = (1 << h2) - 1, nn3 = (1 << h3) - 1;
    if (lane < nn2) {
        t = Tail{base2 + lane, h2, true};
    } else if (nn3 > 0 && lane < nn2 + (nn3 << h2)) {
        const int q = lane - nn2, c = q / nn3;
        t = Tail{base3 + (c << h3) + (q - c * nn3), h2 + h3, true};
    }
    return t;
}

// The one-token build (R1G) folds the second round into the tail as well when the plan has three rounds whose last
// two take at most 6 levels (the reference's trained shapes: D = 10, rounds 4, 3, 3): one dependent global round per
// routed layer instead of two.
__device__ __forceinline__ bool tail_fold(const YggDevModel &m) {
    return m.n_rounds == 3 && m.round_h[1] + m.round_h[2] <= 6;
}

// The deep descent -> leaf index. W0/th0 as in descend; W1 the layer's LDS second-round rows (R1G: the layer's rows of
// the second round in global memory, from slot 2^h0) and th2 this lane's four second-round thresholds (slots
// 2^h0 + 4 lane .. + 3 of the token's row); qb the state below (LDS) for the tail's whole-row dots. hook() runs once,
// while the tail round's loads are in flight (or after the descent).
template <int N, class Hook = NoHook, bool R1G = false>
__device__ __forceinline__ int descend_deep(const YggDevModel &m, const YggDevLayer &y, const int8_t *W0, float th0,
                                            const int8_t *W1, const float4 &th2, const uint32_t (&qbw)[Fast<N>::QW],
                                            const int8_t *qb, float rho, int x, int lane, const Tail &tl,
                                            Hook hook = Hook()) {
    using F = Fast<N>;
    const int qk = lane & 3, qj = lane >> 2;
    const int h0 = m.round_h[0], nn1 = (1 << h0) - 1;
    int ix;
    {
        int dot = 0;
        if (qj < nn1) {
            uint32_t wv[F::QW];
            quad_share<N>(wv, W0 + qj * kLdsRow<N>, qk);
#pragma unroll
            for (int i = 0; i < F::QW; i++) dot = dot4(wv[i], qbw[i], dot);
        }
        dot = sum4(dot);
        const bool right = (float)dot * rho > th0;
        const int loc = walk_round(lane_mask(right && qk == 0 && qj < nn1), h0);
        ix = (1 << h0) + (loc - nn1);
    }
    const bool fold = R1G && tail_fold(m);
    if (!fold) {
        {
            const int h = m.round_h[1], nn = (1 << h) - 1;
            const int sl = ((ix - (1 << h0)) << h) + qj;          // slot within the second round's slots
            uint32_t wv[F::QW];
            if (qj < nn) {
                if constexpr (R1G) quad_share<N>(wv, W1 + (size_t)sl * N, qk);
                else quad_share_r2<N>(wv, W1 + sl * N, qk, sl);
            }
            // slot sl's threshold is component sl & 3 of lane sl >> 2's th2 (sl < 256)
            const int src = (sl >> 2) & 63;
            const float a = __shfl(th2.x, src), b = __shfl(th2.y, src), c = __shfl(th2.z, src), d = __shfl(th2.w, src);
            const int k = sl & 3;
            const float th = k == 0 ? a : (k == 1 ? b : (k == 2 ? c : d));
            int dot = 0;
            if (qj < nn) {
#pragma unroll
                for (int i = 0; i < F::QW; i++) dot = dot4(wv[i], qbw[i], dot);
            }
            dot = sum4(dot);
            const bool right = (float)dot * rho > th;
            const int loc = walk_round(lane_mask(right && qk == 0 && qj < nn), h);
            ix = (ix << h) + (loc - nn);
        }
        if (m.n_rounds == 2) {
            hook();
            return ix - m.E;
        }
    }
    {
        const int r0 = fold ? 1 : 2, d0 = fold ? h0 : h0 + m.round_h[1];   // the tail's first round, levels before it
        const float *thr = y.thr + (size_t)x * y.thr_stride;
        const int slot = tl.ta + ((ix - (1 << d0)) << tl.tsh);
        uint32_t rw[N / 4];
        float th = 0.0f;
        if (tl.on) {
            load_words<N / 4, 16>(rw, y.w + (size_t)slot * N);
            th = thr[slot];
        }
        hook();
        uint32_t qf[N / 4];
        load_words<N / 4, 16>(qf, qb);
        int dot = 0;
#pragma unroll
        for (int i = 0; i < N / 4; i++) dot = dot4(rw[i], qf[i], dot);
        const unsigned long long mask = lane_mask(tl.on && (float)dot * rho > th);
        const int h2 = m.round_h[r0], nn2 = (1 << h2) - 1;
        const int c = walk_bits(mask, h2) - nn2;
        ix = (ix << h2) + c;
        if (m.n_rounds == r0 + 2) {
            const int h3 = m.round_h[r0 + 1], nn3 = (1 << h3) - 1;
            ix = (ix << h3) + (walk_bits(mask >> (nn2 + c * nn3), h3) - nn3);
        }
    }
    return ix - m.E;
}

// the expert's whole gather record and table row, in one burst
// MZ: the model has group scales (the expert's readout row scales, in every layer). UW = false: not U' (its user
// has the layer-input term from elsewhere)
// FACT, routed: U_r's first K4 dwords per coordinate (K4 = input rank / 4), c_r and su_r instead of the table row
// PART: 0 all of it, 1 what the update reads (A16, U', the table row), 2 what the readout reads (P, the row scale)
template <class SH, bool MZ = false, bool UW = true, bool FACT = false, int PART = 0>
__device__ __forceinline__ void gather(Gather<SH, FACT> &G, const YggDevLayer &y, int r, int x, bool routed, int lane,
                                       int K4 = 0) {
    using F = SH;
    // a layer's records and tables lie within 4 GiB (checked at load): 32-bit offsets
    const uint8_t *g = y.gath + (uint32_t)r * (uint32_t)y.gath_bytes;
    if (PART != 2 && lane < F::NL) {
#pragma unroll
        for (int c = 0; c < F::NA; c++) {
            const uint4 v = *(const uint4 *)(g + (c * F::NL + lane) * 16);
            G.aw[4 * c] = v.x; G.aw[4 * c + 1] = v.y; G.aw[4 * c + 2] = v.z; G.aw[4 * c + 3] = v.w;
        }
        if (UW && routed) {
#pragma unroll
            for (int k4 = 0; k4 < F::K4; k4++) {
                uint32_t tmp[F::C];
                load_words<F::C, 4 * F::C>(tmp, g + y.off_U + ((k4 * F::NL + lane) * F::C) * 4);
#pragma unroll
                for (int c = 0; c < F::C; c++) G.uw[k4][c] = tmp[c];
            }
        }
        const int16_t *tr = y.table + ((uint32_t)r * (uint32_t)y.table_sr + (uint32_t)x * (uint32_t)y.table_sx) +
                            F::C * lane;
        if (FACT && routed) tr = (const int16_t *)(g + y.off_FB) + F::C * lane;     // c_r in the record
        if constexpr (F::C == 1) {
            G.trw[0] = tr[0];
        } else {
#pragma unroll
            for (int c = 0; c < F::C / 2; c++) G.trw[c] = (int)((const uint32_t *)tr)[c];
        }
        if constexpr (FACT) {
#pragma unroll
            for (int k4 = 0; k4 < kFactK4; k4++) {
                uint32_t tmp[F::C];
#pragma unroll
                for (int c = 0; c < F::C; c++) tmp[c] = 0u;
                if (routed && k4 < K4) load_words<F::C, 4 * F::C>(tmp, g + y.off_F + ((k4 * F::NL + lane) * F::C) * 4);
#pragma unroll
                for (int c = 0; c < F::C; c++) G.fw[k4][c] = tmp[c];
            }
        }
    }
    if constexpr (FACT) G.fs = routed ? *(const float *)(g + y.off_FS) : 0.0f;
    if constexpr (PART == 1) return;
    // (a model with group scales has the row scales in every layer; without, the readout scale is the layer's)
    if constexpr (MZ) G.mzr = y.mz[(uint32_t)r * SH::R + lane / SH::RL];
    else G.mzr = 0.0f;
    const uint8_t *pp = g + y.off_P;
#pragma unroll
    for (int gi = 0; gi < F::SP / F::GP; gi++) {
        uint32_t tmp[F::GP / 4];
        load_words<F::GP / 4, F::GP>(tmp, pp + (gi * 64 + lane) * F::GP);
#pragma unroll
        for (int i = 0; i < F::GP / 4; i++) G.pw[gi * (F::GP / 4) + i] = tmp[i];
    }
}

// zl[k] = clamp(rint((f32(V'_k . q_below) m_v[k]) rho), +-127) into LDS (cpu/ygg.cpp:285-296); V0 and mv0 are the
// layer's V' rows and m_v in LDS
template <class SH>
__device__ __forceinline__ void layer_input(int8_t *zls, const int8_t *V0, const float *mv0,
                                            const uint32_t (&qbw)[Fast<SH::N>::QW], float rho, int lane) {
    constexpr int N = SH::N;
    using F = Fast<N>;
    const int qk = lane & 3, qj = lane >> 2;
    // pass p: quad j takes row 16 p + j
#pragma unroll
    for (int p = 0; p < SH::RG; p++) {
        const int k = 16 * p + qj;
        uint32_t vv[F::QW];
        quad_share<N>(vv, V0 + k * kLdsRow<N>, qk);
        int a = 0;
#pragma unroll
        for (int i = 0; i < F::QW; i++) a = dot4(vv[i], qbw[i], a);
        a = sum4(a);
        if (qk == 0) {
            float zf = (float)a * mv0[k];
            zf = zf * rho;
            zls[k] = (int8_t)clamp127(cvt_rne(zf));
        }
    }
}

// layer_input with V' in registers: vr[p] the quad share of row 16 p + qj (loaded once by load_vrows)
template <class SH>
__device__ __forceinline__ void load_vrows(uint32_t (&vr)[SH::RG > 0 ? SH::RG : 1][Fast<SH::N>::QW], const YggDevLayer &y,
                                          int lane) {
    constexpr int N = SH::N;
    const int qk = lane & 3, qj = lane >> 2;
#pragma unroll
    for (int p = 0; p < SH::RG; p++) quad_share<N>(vr[p], y.vl + (size_t)(16 * p + qj) * N, qk);
}
template <class SH>
__device__ __forceinline__ void layer_input_regs(int8_t *zls, const uint32_t (&vr)[SH::RG > 0 ? SH::RG : 1][Fast<SH::N>::QW],
                                                 const float *mv0, const uint32_t (&qbw)[Fast<SH::N>::QW], float rho,
                                                 int lane) {
    using F = Fast<SH::N>;
    const int qk = lane & 3, qj = lane >> 2;
#pragma unroll
    for (int p = 0; p < SH::RG; p++) {
        const int k = 16 * p + qj;
        int a = 0;
#pragma unroll
        for (int i = 0; i < F::QW; i++) a = dot4(vr[p][i], qbw[i], a);
        a = sum4(a);
        if (qk == 0) {
            float zf = (float)a * mv0[k];
            zf = zf * rho;
            zls[k] = (int8_t)clamp127(cvt_rne(zf));
        }
    }
}

// this lane's share of expert r's U' (the layout the gather record holds) and its products with zl
template <class SH>
__device__ __forceinline__ void load_uw(uint32_t (&uw)[SH::K4A][SH::C], const YggDevLayer &y, int r, int lane) {
    using F = SH;
    const uint8_t *g = y.gath + (uint32_t)r * (uint32_t)y.gath_bytes + y.off_U;
    const int ln = lane < F::NL ? lane : F::NL - 1;
#pragma unroll
    for (int k4 = 0; k4 < F::K4; k4++) {
        uint32_t tmp[F::C];
        load_words<F::C, 4 * F::C>(tmp, g + ((k4 * F::NL + ln) * F::C) * 4);
#pragma unroll
        for (int c = 0; c < F::C; c++) uw[k4][c] = tmp[c];
    }
}
template <class SH>
__device__ __forceinline__ void uw_products(int (&d)[SH::C], const uint32_t (&uw)[SH::K4A][SH::C], const int8_t *zls) {
#pragma unroll
    for (int c = 0; c < SH::C; c++) d[c] = 0;
#pragma unroll
    for (int k4 = 0; k4 < SH::K4; k4++) {
        const uint32_t zw = ((const uint32_t *)zls)[k4];
#pragma unroll
        for (int c = 0; c < SH::C; c++) d[c] = dot4(uw[k4][c], zw, d[c]);
    }
}

// new state rows of this lane: sat8(((A16 q_old + 2^(s-1)) >> s) + T_r[x] + rint(f32(U'_r zl) m_ul))
// (cpu/ygg.cpp:311-389); qold is the layer's state before the token (LDS). A row is stored as hi and lo signed bytes
// with A16 = 256 hi + lo, so A16 q = 256 (hi q) + (lo q) exactly, two v_dot4 chains on the raw int8 state.
// MUL: per-coordinate layer-input scales at mul (group scales; LDS), else the layer's one scale. PRE: the products
// U'_r zl of this lane's coordinates come computed, at dpre (LDS), instead of from G.uw and zls
// FACT, routed: the input is rint(f32(U_r v[x]) f32(su_r mT_i)) + c_r (cpu/ygg.cpp:339-358) instead of the table row;
// vx the token's code v[x] (K4 dwords, the same for every lane)
template <class SH, bool MUL = false, bool PRE = false, bool FACT = false>
__device__ __forceinline__ void update(int (&qn)[SH::C], const Gather<SH, FACT> &G, const int8_t *qold,
                                       const int8_t *zls, const YggDevLayer &y, bool routed, int shift, int lane,
                                       const float *mul = nullptr, const int *dpre = nullptr,
                                       const uint32_t *vx = nullptr, int K4 = 0) {
    using F = SH;
    constexpr int BLK = F::BLK, C = F::C, RW = BLK / 4;     // dwords of one row's hi (and of its lo) bytes
    const int blk0 = (C * lane / BLK) * BLK;
    uint32_t qv[RW];
    load_words<RW, BLK>(qv, qold + blk0);
    int acc[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        int a = 0;
#pragma unroll
        for (int i = 0; i < RW; i++) a = dot4(G.aw[c * 2 * RW + i], qv[i], a);
        a <<= 8;
#pragma unroll
        for (int i = 0; i < RW; i++) a = dot4(G.aw[c * 2 * RW + RW + i], qv[i], a);
        int in = table_entry(G, c);
        if constexpr (FACT) {
            if (routed) {
                int d = 0;
#pragma unroll
                for (int k4 = 0; k4 < kFactK4; k4++)
                    if (k4 < K4) d = dot4(G.fw[k4][c], vx[k4], d);
                const float fm = G.fs * y.mT[F::C * lane + c];
                in = wadd(cvt_rne((float)d * fm), in);
            }
        }
        acc[c] = wadd((a + (1 << (shift - 1))) >> shift, in);
    }
    if (F::R2 > 0 && routed) {        // (no layer input at rank 0, cpu/ygg.cpp:360)
        int d[C];
        if constexpr (PRE) {
#pragma unroll
            for (int c = 0; c < C; c++) d[c] = dpre[C * lane + c];
        } else {
#pragma unroll
            for (int c = 0; c < C; c++) d[c] = 0;
#pragma unroll
            for (int k4 = 0; k4 < F::K4; k4++) {
                const uint32_t zw = ((const uint32_t *)zls)[k4];
#pragma unroll
                for (int c = 0; c < C; c++) d[c] = dot4(G.uw[k4][c], zw, d[c]);
            }
        }
#pragma unroll
        for (int c = 0; c < C; c++)
            acc[c] = wadd(acc[c], cvt_rne((float)d[c] * (MUL ? mul[C * lane + c] : y.layer_input_scale)));
    }
#pragma unroll
    for (int c = 0; c < C; c++) qn[c] = sat8(acc[c]);
}

// zq[j] = clamp(rint(f32(P_r q) m_z), +-127) into LDS (cpu/ygg.cpp:395-420); pw the lane's P granules, qnew the new
// state (LDS)
template <class SH>
__device__ __forceinline__ void readout(int8_t *zqs, const uint32_t (&pw)[SH::SPW], const int8_t *qnew,
                                        float readout_scale, int lane) {
    using F = SH;
    const int rj = lane / F::RL, rk = lane % F::RL;
    uint32_t qv[F::SPW];
    load_words<F::SPW, F::SPA>(qv, qnew + rk * F::SP);
    int z = 0;
#pragma unroll
    for (int i = 0; i < F::SPW; i++) z = dot4(pw[i], qv[i], z);
    z = group_sum<F::RL>(z);
    if (rk == 0) zqs[rj] = (int8_t)clamp127(cvt_rne((float)z * readout_scale));
}

// f32(Q zq) s_q for the 4 classes of this lane (cpu/ygg.cpp:421-434); Qs the layer's Q planes. SQ: per-class
// scales at sq (group scales; LDS), else scale
template <int R, bool SQ = false>
__device__ __forceinline__ void unembed_terms(float (&term)[4], const int8_t *zqs, const int8_t *Qs, float scale,
                                              int lane, const float *sq = nullptr) {
    constexpr int QC = R / 4, RW = R / 4;              // 16-byte chunks per lane, dwords per class
    uint32_t zw[RW];
    load_words<RW, 16>(zw, zqs);
    uint32_t qq[4 * QC];
#pragma unroll
    for (int p = 0; p < QC; p++) {
        uint32_t q[4];
        load_words<4, 16>(q, Qs + 1024 * p + 16 * lane);
#pragma unroll
        for (int i = 0; i < 4; i++) qq[4 * p + i] = q[i];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        int d = 0;
#pragma unroll
        for (int i = 0; i < RW; i++) d = dot4(qq[u * RW + i], zw[i], d);
        term[u] = (float)d * (SQ ? sq[4 * lane + u] : scale);
    }
}

template <int N>
__device__ __forceinline__ unsigned long long digest_term(const int (&qn)[Fast<N>::C], int r, int l, int lane) {
    using F = Fast<N>;
    static_assert(N <= 256, "sum (q_i + 1)(2 i + 1) <= 256 N^2 must fit 32 bits");
    // sum_i (q_i + 1)(2 i + 1) K mod 2^64 = K sum_i (q_i + 1)(2 i + 1) mod 2^64, and the integer sum is exact in 32
    // bits: the coordinate multiplier K is applied once, after the wavefront sum
    uint32_t a = 0;
    if (lane < F::NL) {
#pragma unroll
        for (int c = 0; c < F::C; c++) a += ((uint8_t)qn[c] + 1u) * (uint32_t)(2 * (F::C * lane + c) + 1);
    }
    a = wave_sum_u32(a);
    return (unsigned long long)(uint32_t)r * kDigestLeaf + (unsigned long long)a * kDigestCoord +
           (unsigned long long)l;
}

__device__ __forceinline__ void store_logits(float *o, const float (&lg)[4], int V, int lane) {
    if ((V & 3) == 0 && 4 * lane + 3 < V) {
        *(float4 *)(o + 4 * lane) = make_float4(lg[0], lg[1], lg[2], lg[3]);
    } else {
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (4 * lane + u < V) o[4 * lane + u] = lg[u];
    }
}

}  // namespace ygg
#include "ygg_kernel_spec.h"
namespace ygg {

// ----------------------------------------------------------------------------------------------- fast_kernel

// MODE: kModeRun (logits, leaves, states), kModeScore (also the digest and the NLL: their constants and lane terms
// take registers the other modes keep for streams) or kModeGenerate (sample the next input from the logits of every
// token, io.gen, instead of reading it from tokens); kModeOne: kModeRun with the deep descent for calls of one token
// (one stream per workgroup, the second round's rows from global memory: nothing staged beyond the usual tables);
// kModeGenOne: kModeGenerate with kModeOne's descent, for models with no DEEP build; kModeGenSpec: kModeGenOne for one
// stream with speculating helper workgroups (ygg_kernel_spec.h; workgroup 0 runs the stream). DEEP: one
// stream per workgroup with the deep descent (generation for few streams), else 4 streams per workgroup with
// descend. CAP (not DEEP): at most 128 VGPRs, 4 wavefronts per SIMD (the most streams resident, some registers
// spilled), else up to 256 (no spills; for calls whose streams all fit at the lower occupancy).
// GROUP: the model has group scales (the tables of GroupTables and the experts' readout row scales)
// FACT: the model stores its routed inputs factored (fact_kernel); only with DEEP = false
template <int N, int R, int R2, int L, int MODE, bool DEEP, bool CAP, bool GROUP, bool FACT, int BLK = 16>
__device__ __forceinline__ void fast_body(const YggDevModel &m, const int32_t *__restrict__ tokens, int B, int T,
                                          int8_t *__restrict__ state, const YggIO &io) {
    float *__restrict__ logits = io.logits;
    int32_t *__restrict__ leaves = io.leaves;
    int8_t *__restrict__ states = io.states;
    unsigned long long *__restrict__ digest = io.digest;
    const int32_t *__restrict__ targets = io.targets;
    double *__restrict__ nll = io.nll;
    using SH = Shape<N, R, R2, BLK>;
    using F = SH;
    // one stream per workgroup for the builds of few streams (DEEP, kModeOne, kModeGenOne): a stream's loads then
    // have a CU's memory path to themselves
    constexpr bool SPEC = MODE == kModeGenSpec;
    constexpr int W = (DEEP || MODE == kModeOne || MODE == kModeGenOne || SPEC) ? 1 : kFastWaves, LR = L > 1 ? L - 1 : 1;
    constexpr bool GEN = MODE == kModeGenerate || MODE == kModeGenOne || SPEC, SCORE = MODE == kModeScore;
    // the deep descent (DEEP: second round in LDS)
    constexpr bool DD = DEEP || MODE == kModeOne || MODE == kModeGenOne || SPEC;
    // SPEC: the routed layers whose descent the helpers take over; every wavefront's state rows (a helper's: the new and
    // the old states of those layers) and slot tail (ygg_kernel_spec.h)
    constexpr int SPS = SPEC ? kSpecDepth<L> : 1;
    using SLY = SpecLayout<SH, SPS>;
    constexpr int QB = (SPEC && 2 * SPS > L ? 2 * SPS : L) * N;
    __shared__ __attribute__((aligned(16))) SharedTables<SH, L> S;
    __shared__ __attribute__((aligned(16))) GroupTablesOf<SH, L, GROUP> GT;
    __shared__ __attribute__((aligned(16))) int8_t W1s[DEEP ? LR : 1][DEEP ? kR2Slots<N> * N : 16];
    __shared__ __attribute__((aligned(16))) int8_t qsw[SPEC ? kFastWaves : W][QB];
    __shared__ __attribute__((aligned(16))) int8_t zlw[W][SH::ZL];
    __shared__ __attribute__((aligned(16))) int8_t zqw[W][SH::ZQ];
    __shared__ __attribute__((aligned(16))) int8_t spw[SPEC ? kFastWaves : 1][SPEC ? SLY::TB : 16];
    // the one-token build without group scales stages its tables layer by layer (load_tables_units): the count of
    // staged units, set to 0 before the one barrier every wavefront meets, at entry
    constexpr bool UNITS = MODE == kModeOne && !GROUP;
    __shared__ uint32_t stage_done;

    // the wavefront index, stream, tokens and leaves are uniform over a wavefront: kept in scalar registers. With one
    // stream per workgroup (W = 1) wavefronts 1-3 stage the LDS tables and then leave.
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    if constexpr (SPEC) {
        // workgroups 1 .. io.spec_helpers are helper workgroups (ygg_kernel_spec.h); any others leave at once
        if (blockIdx.x > 0) {
            if ((int)blockIdx.x > io.spec_helpers) return;
            load_tables<SH, L, 64 * kFastWaves>(S, m, tid);
            if constexpr (GROUP) load_group_tables<SH, L, 64 * kFastWaves>(GT, m, tid);
            if constexpr (DEEP) load_round2<N, L, 64 * kFastWaves>(W1s, m, tid);
            __syncthreads();
            const int j = spec_helper_index(blockIdx.x, wv, io.spec_helpers, m.V);
            if (j < 0) return;
            spec_helper<SH, L, GROUP, DEEP>(m, io, T, j, spec_helper_waves(io.spec_helpers, m.V), S, GT, &W1s[0][0],
                                            qsw[wv], spw[wv], lane,
                                            blockIdx.x % kSpecCopies);
            return;
        }
    }
    const int s = blockIdx.x * W + wv;
    const int V = m.V, VP = m.VP;
    const int K4 = FACT ? m.K / 4 : 0;         // factored input rank / 4
    const bool live = wv < W && s < B;
    // The stream's first token and its state are read before the LDS tables are staged, so that their loads overlap
    // (a launch of one token would otherwise wait for them one after the other).
    const int32_t *tok = tokens + (size_t)s * (GEN ? 1 : T);
    // (measured: the generation kernels run slower with it, 15% with DEEP; one-token launches faster)
    if constexpr (!DEEP && MODE != kModeGenOne && !SPEC) touch_args<L>(m);
    if constexpr (UNITS) {
        // (an LDS-only barrier: global loads issued before it stay in flight)
        if (tid == 0) stage_done = 0u;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    int x_next = (live && T > 0) ? __builtin_amdgcn_readfirstlane(tok[0]) : 0;
    int8_t *st = state + (size_t)s * L * N;
    constexpr int SB = (L * N + 63) / 64;     // state bytes per lane
    int sb[SB];
#pragma unroll
    for (int k = 0; k < SB; k++) sb[k] = (live && lane + 64 * k < L * N) ? st[lane + 64 * k] : 0;
    if constexpr (W == 1) {
        // one stream per workgroup: wavefronts 1-3 stage the LDS tables while the stream's wavefront starts its first
        // token (its own load, then the token layer's record); that one waits for them at a workgroup barrier just
        // before it first reads them, ahead of the first token's first update. Every wavefront meets exactly one
        // barrier, whatever the number of tokens
        if (wv > 0) {
            if constexpr (UNITS) {
                load_tables_units<SH, L, 64 * (kFastWaves - 1)>(S, m, tid - 64, &stage_done);
                return;
            }
            load_tables<SH, L, 64 * (kFastWaves - 1)>(S, m, tid - 64);
            if constexpr (GROUP) load_group_tables<SH, L, 64 * (kFastWaves - 1)>(GT, m, tid - 64);
            if constexpr (DEEP) load_round2<N, L, 64 * (kFastWaves - 1)>(W1s, m, tid - 64);
            __syncthreads();
            // SPEC: then helpers on the stream's own CU
            if constexpr (SPEC)
                spec_helper<SH, L, GROUP, DEEP>(m, io, T, io.spec_helpers + spec_pairs(io.spec_helpers, m.V) + wv - 1,
                                                spec_helper_waves(io.spec_helpers, m.V), S, GT, &W1s[0][0], qsw[wv],
                                                spw[wv], lane, 0);
            return;
        }
    } else {
        load_tables<SH, L, 64 * kFastWaves>(S, m, tid);
        if constexpr (GROUP) load_group_tables<SH, L, 64 * kFastWaves>(GT, m, tid);
        __syncthreads();
    }
    if (!live) return;

    Tail tl{};
    if constexpr (DD) tl = make_tail(m, lane, (!DEEP && tail_fold(m)) ? 1 : 2);
    const int n2 = m.n_rounds > 1 ? 1 << (m.round_h[0] + m.round_h[1]) : 0;   // second-round slots
    int8_t *qs = qsw[wv];
    int8_t *zls = zlw[wv];
    int8_t *zqs = zqw[wv];
    const int qj = lane >> 2;
    const int nn1 = (1 << m.round_h[0]) - 1;

#pragma unroll
    for (int k = 0; k < SB; k++)
        if (lane + 64 * k < L * N) qs[lane + 64 * k] = (int8_t)sb[k];
    if (lane < SH::ZL) zls[lane] = 0;
    wave_sync();
    unsigned long long dg = (SCORE && digest) ? digest[s] : 0ull;
    NllSum nacc;
    // W = 1: the stream's wavefront has met the barrier that waits for the LDS tables (UNITS: met at entry; it waits
    // for each routed layer's tables before that layer's descent)
    bool staged = W > 1 || UNITS;
    // SPEC: steps taken from the helpers' slots and computed here, whether the last one was taken
    int spec_hits = 0, spec_misses = 0;
    bool spec_prev = true;
    int8_t *const sps = spw[0];
    // SPEC: the output bias, loaded once (the wait for a load issued after a store waits for the store too); the
    // sampled tokens, written 64 at a time (lane t % 64 holds step t's), so that no such store waits ahead of a slot's
    // look
    float bias[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        bias[u] = (SPEC && 4 * lane + u < VP) ? m.output_bias[4 * lane + u] : 0.0f;
        // (waited for here: a load still in flight at the loop's entry would be waited for, with every later one, in
        // the loop)
        if constexpr (SPEC) asm volatile("" : "+v"(bias[u]));
    }
    int gen_held = 0, sampled = 0;
    // SPEC: the first step's input for its helpers
    if constexpr (SPEC)
        if (T >= 2 && x_next >= 0 && x_next < V) spec_token(io, 0, x_next, lane);

    const int lane_out = lane;
    for (int t = 0; t < T; t++) {
        // SPEC at d_state 256: the lane index made opaque at each step, so that every layer's per-lane addresses are
        // formed in the step instead of hoisted out of the loop and kept live (that shape's stream spilled them to
        // scratch: 536 -> 368 bytes, 10.5 -> 9.8 us per generated token; the narrower shapes, which do not spill
        // them, lost 1-8% with it)
        int lane_in = lane_out;
        if constexpr (SPEC && N > 128) asm volatile("" : "+v"(lane_in));
        const int lane = lane_in;
        const int x = x_next;
        if (!GEN && t + 1 < T) x_next = __builtin_amdgcn_readfirstlane(tok[t + 1]);
        if (x < 0 || x >= V) {
            if (lane == 0) atomicOr(m.err, 1u);
            break;
        }
        // thresholds of the first router round of every routed layer (SPEC: issued after the slot's poll, behind the
        // slot's record: loads issued before the poll's loop are waited for, at their use, with every later load and
        // store)
        float th1[LR];
        // DEEP: and those of the second round, four per lane (components in separate arrays, which the selects
        // below keep in registers)
        float th2x[LR], th2y[LR], th2z[LR], th2w[LR];
        auto load_thresholds = [&]() {
#pragma unroll
            for (int l = 1; l < L; l++)
                th1[l - 1] = qj < nn1 ? m.layers[l].thr[(size_t)x * m.layers[l].thr_stride + qj] : 0.0f;
#pragma unroll
            for (int l = 1; l < L; l++) {
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (DD && 4 * lane < n2)
                    v = *(const float4 *)(m.layers[l].thr + (size_t)x * m.layers[l].thr_stride +
                                          (1 << m.round_h[0]) + 4 * lane);
                th2x[l - 1] = v.x; th2y[l - 1] = v.y; th2z[l - 1] = v.z; th2w[l - 1] = v.w;
            }
        };
        if constexpr (!SPEC) load_thresholds();
        // SPEC: x's slot, which holds this step's layers 0 .. SPS - 1 and layer SPS's leaf and layer input (a short
        // wait after a step that had its slot, a single look after one that did not)
        bool hit = false;
        Gather<SH, FACT> Gs;       // SPEC with the slot: layer SPS's record, gathered as soon as its leaf is known
        int rs = 0;
        if constexpr (SPEC) {
            if (t > 0) {
                hit = __builtin_amdgcn_readfirstlane(
                          (int)spec_take<SH, SPS>(io, x, t, qs, sps, lane, spec_prev ? 400 : 30, rs)) != 0;
                spec_prev = hit;
                spec_hits += hit ? 1 : 0;
                spec_misses += hit ? 0 : 1;
                // (a slot is taken only with every unit of this step: its leaf is one a helper found; the mask keeps
                // the record address in the layer whatever the word holds)
                rs &= m.E - 1;
                if (hit) gather<SH, GROUP, true, FACT>(Gs, m.layers[SPS], rs, x, true, lane, K4);
            }
            load_thresholds();
        }
        float lg[4];
#pragma unroll
        for (int u = 0; u < 4; u++) lg[u] = SPEC ? bias[u] : (4 * lane + u < VP ? m.output_bias[4 * lane + u] : 0.0f);
        // SPEC with the slot: the unembedding terms of layers 0 .. SPS - 1 from its readouts, in layer order
        if constexpr (SPEC) {
            if (hit && 4 * lane < VP) {
#pragma unroll
                for (int l = 0; l < SPS; l++) {
                    float term[4];
                    const float *sq = nullptr;
                    if constexpr (GROUP) sq = GT.sq[l];
                    unembed_terms<R, GROUP>(term, sps + l * R, S.Q[l], m.layers[l].unembed_scale, lane, sq);
#pragma unroll
                    for (int u = 0; u < 4; u++) lg[u] = lg[u] + term[u];
                }
            }
        }

        // The readout of layer l (P_r q -> zq -> Q zq into the logits) is not on the path to layer l + 1, which needs
        // only the new state: it runs while the loads of layer l + 1's first global router round are in flight
        // (pl: the layer whose readout is pending, ppw: its P granules). The logits still add layer by layer in order.
        uint32_t ppw[F::SPW];
        float pmz = 0.0f;
        int pl = -1;
        auto flush = [&]() {
            if (pl >= 0) {
                const YggDevLayer &yp = m.layers[pl];
                readout<SH>(zqs, ppw, qs + pl * N, GROUP ? pmz : yp.readout_scale, lane);
                wave_sync();
                if (4 * lane < VP) {
                    float term[4];
                    const float *sq = nullptr;
                    if constexpr (GROUP) sq = GT.sq[pl];
                    unembed_terms<R, GROUP>(term, zqs, S.Q[pl], yp.unembed_scale, lane, sq);
#pragma unroll
                    for (int u = 0; u < 4; u++) lg[u] = lg[u] + term[u];
                }
                wave_sync();
                pl = -1;
            }
        };

        // not unrolled: an unrolled loop keeps every layer's pointers in scalar registers at once and spills them
        // (the first layer taken through readfirstlane: a per-lane index would read every layer's fields with vector
        // loads)
        const int l0 = __builtin_amdgcn_readfirstlane((SPEC && hit) ? SPS : 0);
#pragma unroll 1
        for (int l = l0; l < L; l++) {
            const YggDevLayer &y = m.layers[l];
            int r = x;
            float rho = 0.0f;
            uint32_t qbw[F::QW];
            // SPEC, the slot's layer: leaf, layer input and record as taken above
            const bool given = SPEC && hit && l == SPS;
            if (given) r = rs;
            if (l > 0 && !given) {
                if constexpr (UNITS) stage_wait(&stage_done, (uint32_t)((kFastWaves - 1) * (l + 1)), m.err, lane);
                float th = th1[0];
#pragma unroll
                for (int i = 1; i < LR; i++) th = l - 1 == i ? th1[i] : th;
                rho = below_and_rho<N>(qbw, qs + (l - 1) * N, y.rms_eps, lane);
                if constexpr (GROUP)
                    if (y.r2b) rho = group_rho<N>(qbw, GT.r2[l - 1], y.rms_eps);
                if constexpr (!DD) {
                    r = descend<N>(m, y, S.W[l - 1], th, qbw, rho, x, lane, flush);
                } else {
                    float4 t2 = make_float4(th2x[0], th2y[0], th2z[0], th2w[0]);
#pragma unroll
                    for (int i = 1; i < LR; i++) {
                        const bool b = l - 1 == i;
                        t2.x = b ? th2x[i] : t2.x;
                        t2.y = b ? th2y[i] : t2.y;
                        t2.z = b ? th2z[i] : t2.z;
                        t2.w = b ? th2w[i] : t2.w;
                    }
                    if constexpr (DEEP)
                        r = descend_deep<N>(m, y, S.W[l - 1], th, W1s[DEEP ? l - 1 : 0], t2, qbw, qs + (l - 1) * N,
                                            rho, x, lane, tl, flush);
                    else
                        r = descend_deep<N, decltype(flush), true>(m, y, S.W[l - 1], th,
                                                                   y.w + ((size_t)1 << m.round_h[0]) * N, t2, qbw,
                                                                   qs + (l - 1) * N, rho, x, lane, tl, flush);
                }
            }
            // (SPEC: the slot layer's record and every later one in the same registers: a separate copy would stay
            // live through the loop)
            Gather<SH, FACT> Gl;
            Gather<SH, FACT> &G = SPEC ? Gs : Gl;
            if (!given) gather<SH, GROUP, true, FACT>(G, y, r, x, l > 0, lane, K4);
            if constexpr (W == 1)
                if (!staged) {      // the LDS tables staged (see above)
                    __syncthreads();
                    staged = true;
                }
            if (l > 0 && !given) layer_input<SH>(zls, S.V[l - 1], S.mv[l - 1], qbw, rho, lane);
            wave_sync();
            int qn[F::C];
            const float *mul = nullptr;
            if constexpr (GROUP) mul = GT.mul[l > 0 ? l - 1 : 0];
            const uint32_t *vx = nullptr;
            if constexpr (FACT) vx = (const uint32_t *)(y.vt + (size_t)x * m.K);
            if (lane < F::NL)
                update<SH, GROUP, false, FACT>(qn, G, qs + l * N, given ? sps + SPS * R + 4 : zls, y, l > 0, m.shift,
                                               lane, mul, nullptr, vx, K4);
            wave_sync();
            if (lane < F::NL) {
#pragma unroll
                for (int c = 0; c < F::C; c++) qs[l * N + F::C * lane + c] = (int8_t)qn[c];
            }
            wave_sync();
            // SPEC, step computed here: its states of layers 0 .. SPS - 1 for the next step's helpers
            if constexpr (SPEC)
                if (!hit && l == SPS - 1 && t + 1 < T) spec_publish<SH, SPS>(io, t, x, qs, lane);
            if (leaves && lane == 0) leaves[((size_t)s * T + t) * L + l] = r;
            if (SCORE && digest) dg = dg * kDigestMul + digest_term<N>(qn, r, l, lane);
#pragma unroll
            for (int i = 0; i < F::SPW; i++) ppw[i] = G.pw[i];
            pmz = G.mzr;
            pl = l;
            if (l == L - 1) flush();
        }

        if (logits) store_logits(logits + ((size_t)s * T + t) * V, lg, V, lane);
        if (SCORE && nll) {
            const int yv = targets[(size_t)s * T + t];
            if (yv >= 0 && yv < V) token_nll(nacc, lg, V, yv, lane);
            else if (lane == 0) atomicOr(m.err, 2u);
        }
        if (GEN) {
            x_next = __builtin_amdgcn_readfirstlane(sample_token(lg, V, io.temperature, io.top_k, io.seed, s, t, lane));
            if constexpr (SPEC) {
                // the next step's input for its helpers (steps up to T - 2 have them)
                if (t + 2 < T) spec_token(io, t + 1, x_next, lane);
                if (lane == (t & 63)) gen_held = x_next;
                if ((t & 63) == 63) io.gen[(size_t)s * T + t - 63 + lane] = gen_held;
                sampled = t + 1;
            } else if (lane == 0) {
                io.gen[(size_t)s * T + t] = x_next;
            }
        }
        if (states) {
            int8_t *so = states + ((size_t)s * T + t) * L * N;
            for (int i = lane; i < L * N; i += 64) so[i] = qs[i];
        }
    }
    // (a call that ended before its first update, T = 0 or a first token out of range, still meets the barrier)
    if constexpr (W == 1)
        if (!staged) __syncthreads();
    wave_sync();
    for (int i = lane; i < L * N; i += 64) st[i] = qs[i];
    if constexpr (SPEC) {
        // the sampled tokens after the last whole 64
        const int rest = sampled & 63;
        if (lane < rest) io.gen[(size_t)s * T + sampled - rest + lane] = gen_held;
    }
    if constexpr (SPEC)
        if (lane == 0) {
            spec_count(io.spec, 0, (unsigned long long)spec_hits);
            spec_count(io.spec, 1, (unsigned long long)spec_misses);
        }
    if (SCORE && digest && lane == 0) digest[s] = dg;
    if (SCORE && nll && lane == 0) nll[s] += nacc.value();
}


// (one wave per SIMD for the deep builds and the speculating build, which hold a CU per workgroup: their registers
// spill to AGPRs instead of scratch)
template <int N, int R, int R2, int L, int MODE, bool DEEP, bool CAP, bool GROUP>
__global__ __launch_bounds__(64 * kFastWaves)
__attribute__((amdgpu_waves_per_eu((DEEP || MODE == kModeGenSpec) ? 1 : (CAP ? 4 : 2))))
void fast_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                 const YggIO io) {
    fast_body<N, R, R2, L, MODE, DEEP, CAP, GROUP, false>(m, tokens, B, T, state, io);
}

// fast_kernel for transition blocks of 8 (fast-only shapes: the router, layer input and readout are the same; a
// lane's A16 rows hold 8 hi and 8 lo bytes each)
template <int N, int R, int R2, int L, int MODE, bool CAP, bool GROUP>
__global__ __launch_bounds__(64 * kFastWaves)
__attribute__((amdgpu_waves_per_eu(CAP ? 4 : 2)))
void fast8_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                  const YggIO io) {
    fast_body<N, R, R2, L, MODE, false, CAP, GROUP, false, 8>(m, tokens, B, T, state, io);
}

// fast_kernel for models whose routed layers store their input factored (cpu/ygg.cpp:339-358, input rank <= 64): a
// routed expert's gather record holds U_r, c_r and su_r beside A16, U' and P; the token's code v[x] and the
// coordinate scales mT are read from the layer's arrays
template <int N, int R, int R2, int L, int MODE, bool CAP, bool GROUP>
__global__ __launch_bounds__(64 * kFastWaves)
__attribute__((amdgpu_waves_per_eu(CAP ? 4 : 2)))
void fact_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                 const YggIO io) {
    fast_body<N, R, R2, L, MODE, false, CAP, GROUP, true>(m, tokens, B, T, state, io);
}
// fact_kernel at transition blocks of 8
template <int N, int R, int R2, int L, int MODE, bool CAP, bool GROUP>
__global__ __launch_bounds__(64 * kFastWaves)
__attribute__((amdgpu_waves_per_eu(CAP ? 4 : 2)))
void fact8_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                  const YggIO io) {
    fast_body<N, R, R2, L, MODE, false, CAP, GROUP, true, 8>(m, tokens, B, T, state, io);
}

// ----------------------------------------------------------------------------------------------- pipe_kernel

// CAP: at most 128 VGPRs (4 wavefronts per SIMD: more streams resident, some registers spilled), else as many as
// the kernel needs (no spills: faster for few streams)
// MODE: kModeRun (logits, leaves, states) or kModeScore (also the digest and the NLL, whose constants the run build
// does without: its capped builds then fit 128 VGPRs without spills)
template <int N, int R, int R2, int L, int MODE, bool CAP, bool GROUP>
__global__ __launch_bounds__(64 * L) __attribute__((amdgpu_waves_per_eu(CAP ? 4 : 1)))
void pipe_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                 const YggIO io) {
    // generation needs every layer of a token before the next one; the dispatcher never sends it here
    constexpr bool SCORE = MODE == kModeScore;
    float *__restrict__ logits = io.logits;
    int32_t *__restrict__ leaves = io.leaves;
    int8_t *__restrict__ states = io.states;
    unsigned long long *__restrict__ digest = SCORE ? io.digest : nullptr;
    const int32_t *__restrict__ targets = io.targets;
    double *__restrict__ nll = SCORE ? io.nll : nullptr;
    using SH = Shape<N, R, R2>;
    using F = SH;
    __shared__ __attribute__((aligned(16))) SharedTables<SH, L> S;
    __shared__ __attribute__((aligned(16))) GroupTablesOf<SH, L, GROUP> GT;
    __shared__ __attribute__((aligned(16))) int8_t qbuf[L][2][N];            // layer l after token t: [l][t & 1]
    __shared__ __attribute__((aligned(16))) float lgs[L][256];               // logits of token t: row t % L
    __shared__ __attribute__((aligned(16))) unsigned long long dterm[L][L];  // digest terms of token t: row t % L
    __shared__ __attribute__((aligned(16))) int8_t zlw[L][SH::ZL];
    __shared__ __attribute__((aligned(16))) int8_t zqw[L][SH::ZQ];
    __shared__ int stop_t;                                                   // first token out of range

    // the wavefront's layer and the tokens are uniform over a wavefront: kept in scalar registers
    const int tid = threadIdx.x, l = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int s = blockIdx.x;
    const int V = m.V, VP = m.VP;
    load_tables<SH, L, 64 * L>(S, m, tid);
    if constexpr (GROUP) load_group_tables<SH, L, 64 * L>(GT, m, tid);
    const YggDevLayer &y = m.layers[l];
    int8_t *st = state + ((size_t)s * L + l) * N;
    for (int i = lane; i < N; i += 64) qbuf[l][1][i] = st[i];     // the state before token 0
    if (lane < SH::ZL) zlw[l][lane] = 0;
    if (tid == 0) stop_t = T;
    __syncthreads();

    const int32_t *tok = tokens + (size_t)s * T;
    const int qj = lane >> 2;
    const int nn1 = (1 << m.round_h[0]) - 1;
    unsigned long long dg = (digest && l == L - 1) ? digest[s] : 0ull;
    NllSum nacc;
    // loaded a tick ahead: the first-round thresholds (routed layers) or the gather record (token layer; not for the
    // largest shape, whose two records in flight would spill: the token layer's chain is the shortest anyway)
    constexpr bool kAhead = N * R2 < 256 * 64;
    float th0 = 0.0f;
    Gather<SH> G0;
    if (T > 0) {
        const int x0 = __builtin_amdgcn_readfirstlane(tok[0]);
        if (x0 >= 0 && x0 < V) {
            if (l > 0 && qj < nn1) th0 = y.thr[(size_t)x0 * y.thr_stride + qj];
            if (kAhead && l == 0) gather<SH, GROUP>(G0, y, x0, x0, false, lane);
        }
    }

    for (int k = 0; k < T + L - 1; k++) {
        const int t = k - l;
        if (t >= 0 && t < T && t < stop_t) {
            const int x = __builtin_amdgcn_readfirstlane(tok[t]);
            const bool ok = x >= 0 && x < V;
            if (l == 0 && !ok && lane == 0) {
                atomicOr(m.err, 1u);
                stop_t = t;
            }
            if (ok) {
                int r = x;
                float rho = 0.0f;
                uint32_t qbw[F::QW];
                Gather<SH> G;
                if (l > 0) {
                    rho = below_and_rho<N>(qbw, qbuf[l - 1][t & 1], y.rms_eps, lane);
                    if constexpr (GROUP)
                        if (y.r2b) rho = group_rho<N>(qbw, GT.r2[l - 1], y.rms_eps);
                    r = descend<N>(m, y, S.W[l - 1], th0, qbw, rho, x, lane);
                    gather<SH, GROUP>(G, y, r, x, true, lane);
                    layer_input<SH>(zlw[l], S.V[l - 1], S.mv[l - 1], qbw, rho, lane);
                } else if constexpr (kAhead) {
                    G = G0;
                } else {
                    gather<SH, GROUP>(G, y, x, x, false, lane);
                }
                if (t + 1 < T) {
                    const int xn = __builtin_amdgcn_readfirstlane(tok[t + 1]);
                    if (xn >= 0 && xn < V) {
                        if (l > 0 && qj < nn1) th0 = y.thr[(size_t)xn * y.thr_stride + qj];
                        if (kAhead && l == 0) gather<SH, GROUP>(G0, y, xn, xn, false, lane);
                    }
                }
                wave_sync();
                int qn[F::C];
                if (lane < F::NL) {
                    const float *mul = nullptr;
                    if constexpr (GROUP) mul = GT.mul[l > 0 ? l - 1 : 0];
                    update<SH, GROUP>(qn, G, qbuf[l][(t + 1) & 1], zlw[l], y, l > 0, m.shift, lane, mul);
#pragma unroll
                    for (int c = 0; c < F::C; c++) qbuf[l][t & 1][F::C * lane + c] = (int8_t)qn[c];
                }
                wave_sync();
                readout<SH>(zqw[l], G.pw, qbuf[l][t & 1], GROUP ? G.mzr : y.readout_scale, lane);
                wave_sync();
                float *lr = lgs[t % L];
                if (4 * lane < VP) {
                    float term[4];
                    const float *sq = nullptr;
                    if constexpr (GROUP) sq = GT.sq[l];
                    unembed_terms<R, GROUP>(term, zqw[l], S.Q[l], y.unembed_scale, lane, sq);
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const float base = l == 0 ? m.output_bias[4 * lane + u] : lr[4 * lane + u];
                        lr[4 * lane + u] = base + term[u];
                    }
                }
                if (leaves && lane == 0) leaves[((size_t)s * T + t) * L + l] = r;
                if (states) {
                    int8_t *so = states + (((size_t)s * T + t) * L + l) * N;
                    for (int i = lane; i < N; i += 64) so[i] = qbuf[l][t & 1][i];
                }
                if (digest) {
                    const unsigned long long f = digest_term<N>(qn, r, l, lane);
                    if (lane == 0) dterm[t % L][l] = f;
                }
                if (l == L - 1) {
                    wave_sync();
                    float lg[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? lr[4 * lane + u] : 0.0f;
                    if (logits) store_logits(logits + ((size_t)s * T + t) * V, lg, V, lane);
                    if (nll) {
                        const int yv = targets[(size_t)s * T + t];
                        if (yv >= 0 && yv < V) token_nll(nacc, lg, V, yv, lane);
                        else if (lane == 0) atomicOr(m.err, 2u);
                    }
                    if (digest) {
#pragma unroll
                        for (int j = 0; j < L; j++) dg = dg * kDigestMul + dterm[t % L][j];
                        dg = uniform_u64(dg);
                    }
                }
            }
        }
        __syncthreads();
    }
    const int te = T < stop_t ? T : stop_t;                          // tokens processed
    for (int i = lane; i < N; i += 64) st[i] = qbuf[l][(te + 1) & 1][i];
    if (digest && l == L - 1 && lane == 0) digest[s] = dg;
    if (nll && l == L - 1 && lane == 0) nll[s] += nacc.value();
}


// ----------------------------------------------------------------------------------------------- flow_kernel
// Scoring with the tokens known, one stream per workgroup, as a software pipeline over ticks.
// Of layer l's work on token t only the update is on the layer's own recurrence (q_l(t) needs q_l(t - 1)): the router
// rounds and the gather need just the layer below at the same token. So a routed layer runs as stages, one per router
// round and one for the update, a tick apart: a round's row and threshold loads are issued in one tick and consumed in
// the next, the record a tick before its update, and the ticks are separated by barriers that wait for LDS only, so
// the global loads of every stage stay in flight across them. A tick then costs the stages' arithmetic, not their
// chain of memory round trips (pipe_kernel does each layer's whole chain in one tick).
//
// Waves: the token layer has one; a routed layer a descent wave (its router rounds, the layer input; SPLIT: two, one
// per token parity) and an update wave (the record, the update, the readout); SPLIT builds add the logits wave (and
// at 2 layers the layer-input wave, in score builds the NLL wave). They share the SIMDs' issue slots, placed by a
// table, and so overlap each other's LDS and arithmetic latencies.
//
// Schedule (P router rounds, o_l the tick of layer l's update of token 0): the token layer gathers token t at tick t
// (two record buffers; SB1: one, refilled a tick later) and updates it at tick o_0 + t = 2 + t; routed layer l's
// descent runs round j of token t at tick o_(l-1) + 1 + t + j (round 0 from the LDS rows, its thresholds loaded a tick
// before) and leaves the leaf and the layer input in LDS after round P - 1; its update wave issues the token's record
// the tick after and updates it the tick after that, o_l = o_(l-1) + P + 2. States live in a ring per layer (slot
// (t + 1) mod QR after token t, slot 0 the state before token 0); logits add up layer by layer, in order (in a ring of
// logit rows over the tokens in flight, or the logits wave from the layers' readout rows).
//
// Every stage runs in every tick, on a clamped token and valid tree nodes while the pipeline fills and drains, and
// only its stores are conditional: the registers carried from tick to tick are then written once per tick in
// straight-line code, so the loads that fill them are waited for where the next tick reads them and nowhere else.
// Tokens come through the scalar cache (their wait counter is not the vector loads').
constexpr int kFlowStates = 8;     // state ring slots per layer (> the rounds)
template <int L, int P> constexpr int kFlowLogits = (L - 1) * (P + 2) + 1;   // tokens in flight between layers
constexpr int kFlowToken0 = 2;     // tick of the token layer's update of token 0 (its records issued two ticks ahead)

// BIG: the largest shape, whose 32 KiB record does not fit twice in the update wave's registers: its descent wave
// keeps V' in registers (not LDS) and computes the U'z products itself, handing them over in dring, so the update
// wave's records hold A16, P and the table row only
template <class SH> constexpr bool kFlowBig = SH::N * SH::R2 >= 256 * 64;
// SPLIT (all but BIG; at 5 layers the run builds): two descent wavefronts per routed layer, one for the tokens of each
// parity. A token's rounds run a tick apart, so in every tick each of the two takes every other round (the rounds of
// its tokens) and hands each round's loads to its own next round: half the descent work a wave and tick, no data
// crosses between them. (5-layer score builds: 13 wavefronts would put 4 on a SIMD, a cap of 128 VGPRs, and spill.)
// SPLIT builds also finish the logits on a wavefront of their own (LOGW): each layer's update wave leaves its readout
// row zq of token t in a ring, and a tick after the last layer's update the logits wave adds the bias and every
// layer's unembedding term, in layer order, stores the row and, scoring, adds the NLL and the digest.
template <class SH, int L, bool SC> constexpr bool kFlowSplitSC = !kFlowBig<SH> && (L <= 4 || !SC);
template <class SH, int L, int MODE> constexpr bool kFlowSplit = kFlowSplitSC<SH, L, MODE == kModeScore>;
// LIW (SPLIT builds of 2 layers): the layer inputs on a wavefront of their own (the layer-input wave). The descent
// wave that ran a token's last round leaves its rho in LDS, and a tick later that wave forms the token's layer input
// from the state below (still in its ring), a tick before the update reads it. (Measured at batch 1: configuration 1
// 2.29 -> 1.96 ms; with more layers the extra wavefront lowered residency or crowded a SIMD, and lost.)
template <class SH, int L, int MODE> constexpr bool kFlowLiw = kFlowSplit<SH, L, MODE> && L == 2;
// wavefronts: the token layer's, then per routed layer the descent wave (SPLIT: two) and the update wave (SPLIT: and
// the logits wave; LIW: and the layer-input wave)
template <class SH, int L, int MODE>
constexpr int kFlowWaves = kFlowSplit<SH, L, MODE> ? 3 * L - 1 + (kFlowLiw<SH, L, MODE> ? 1 : 0) : 2 * L - 1;
// VREG: V' in the descent wave's registers (BIG, up to 4 layers: 7 wavefronts leave 256 VGPRs a wave; at 5 layers,
// 9 wavefronts leave 168, and V' stays in LDS)
template <class SH, int L> constexpr bool kFlowVreg = kFlowBig<SH> && 2 * L - 1 <= 8;
// ZQR (BIG at 5 layers, where LDS is short): each layer leaves its zq row of token t in a ring and the last layer's
// update wave adds every layer's unembedding term, in layer order, instead of the layers adding theirs to a ring of
// logit rows
// Score builds of the form with V' in LDS and the SPLIT score builds run the NLL on a wavefront of their own (after
// the other waves): its tick loop holds the double-precision exp and log constants, which in an update wave's loop
// spill beside the record, and its log-sum-exp would otherwise lengthen the tick of the wave finishing the logits.
template <class SH, int L, int MODE>
constexpr bool kFlowNllWave = MODE == kModeScore && ((kFlowBig<SH> && !kFlowVreg<SH, L>) || kFlowSplit<SH, L, MODE>);
template <class SH, int L, int MODE>
constexpr int kFlowThreads = 64 * (kFlowWaves<SH, L, MODE> + (kFlowNllWave<SH, L, MODE> ? 1 : 0));

// SC (score builds): with V' in LDS the finished logits of token t wait in lgs[t & 1] for the NLL wave
template <class SH, int L, int P, bool GROUP, bool SC> struct FlowShared {
    static constexpr bool BIG = kFlowBig<SH>, VREG = kFlowVreg<SH, L>, ZQR = BIG && !VREG;
    static constexpr bool LOGW = kFlowSplitSC<SH, L, SC>, ZQRING = ZQR || LOGW;
    static constexpr int QR = (BIG && P < 4) ? 4 : kFlowStates;           // state ring slots (> P)
    // tokens in flight between the token layer's update and the last reader of their ring slots (LOGW: one tick more)
    static constexpr int LG = kFlowLogits<L, P> + (LOGW ? 1 : 0);
    static constexpr int LGS = (ZQR || LOGW) ? (SC ? 2 : 1) : LG;         // logits slots
    alignas(16) SharedTables<SH, L, !VREG> S;
    alignas(16) GroupTablesOf<SH, L, GROUP> GT;
    alignas(16) int8_t qring[L][QR][SH::N];
    alignas(16) int dring[BIG ? L : 1][2][BIG ? SH::N : 4];               // U'z of token t: [l][t & 1]
    alignas(16) float lgs[LGS][256];
    alignas(16) int8_t zqr[ZQRING ? L : 1][ZQRING ? LG : 1][SH::ZQ];       // ZQR, LOGW: zq of layer l, token t
    alignas(16) unsigned long long dterm[LG][L];
    alignas(16) int8_t zlw[L][4][SH::ZL];                 // layer input of token t: [l][t & 3]
    float rhol[L][4];                                     // LIW: rho of token t's state below, for the layer input
    alignas(16) int8_t zqw[L][SH::ZQ];
    int leafx[L][2][2];                                   // leaf and token of token t: [l][t & 1]
    int stop_t;
};
template <int N, int R, int R2, int L, int P, bool GROUP>
constexpr bool kFlowFits = L >= 2 && sizeof(FlowShared<Shape<N, R, R2>, L, P, GROUP, true>) <= 160 * 1024;

// a wavefront-uniform 32-bit load through the scalar cache, waited for at once (it leaves the vector loads in flight)
__device__ __forceinline__ int scalar_load(const int32_t *p) {
    const unsigned long long a = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a), hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
    const int32_t *q = (const int32_t *)(((unsigned long long)hi << 32) | lo);
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(q) : "memory");
    return v;
}

// the barrier between ticks: LDS writes done and visible, global loads left in flight
__device__ __forceinline__ void flow_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// one router round from the loaded row shares (quad qj holds node qj's dot product): the node index ix at the round's
// start (heap numbering) -> at its end
template <int N>
__device__ __forceinline__ int round_step(const uint32_t (&wv)[Fast<N>::QW], const uint32_t (&qbw)[Fast<N>::QW],
                                          float rho, float th, int ix, int h, int lane) {
    const int qk = lane & 3, qj = lane >> 2, nn = (1 << h) - 1;
    int dot = 0;
#pragma unroll
    for (int i = 0; i < Fast<N>::QW; i++) dot = dot4(wv[i], qbw[i], dot);
    dot = sum4(dot);
    const bool right = (float)dot * rho > th;
    return (ix << h) + (walk_round(lane_mask(right && qk == 0 && qj < nn), h) - nn);
}

// the per-layer outputs of token t (leaf, state, digest term)
template <class SH, int L, int P, bool SCORE, bool GROUP>
__device__ __forceinline__ void flow_outputs(FlowShared<SH, L, P, GROUP, SCORE> &sh, const YggDevModel &m,
                                             const int (&qn)[SH::C], const int8_t *qnew, int l, int t, int r, int s,
                                             int T, const YggIO &io, int lane) {
    constexpr int N = SH::N, LG = FlowShared<SH, L, P, GROUP, SCORE>::LG;
    if (io.leaves && lane == 0) io.leaves[((size_t)s * T + t) * L + l] = r;
    if (io.states) {
        int8_t *so = io.states + (((size_t)s * T + t) * L + l) * N;
        for (int i = lane; i < N; i += 64) so[i] = qnew[i];
    }
    if (SCORE && io.digest) {
        const unsigned long long f = digest_term<N>(qn, r, l, lane);
        if (lane == 0) sh.dterm[t % LG][l] = f;
    }
}

// the last layer completes token t: its logits out, the NLL (or, with V' in LDS, the logits for the NLL wave), the
// digest of every layer's term in layer order
template <class SH, int L, int P, bool SCORE, bool GROUP>
__device__ __forceinline__ void flow_finish(FlowShared<SH, L, P, GROUP, SCORE> &sh, const YggDevModel &m,
                                            const float (&lg)[4], int t, int s, int T, const YggIO &io,
                                            unsigned long long &dg, NllSum &nacc, int lane) {
    using FS = FlowShared<SH, L, P, GROUP, SCORE>;
    constexpr int LG = FS::LG;
    const int V = m.V;
    // (ZQR, LOGW: the NLL wave takes the NLL from the logits row left in lgs)
    constexpr bool ROW = FS::ZQR || FS::LOGW;
    if (SCORE && ROW && io.nll) *(float4 *)(sh.lgs[t & 1] + 4 * lane) = make_float4(lg[0], lg[1], lg[2], lg[3]);
    wave_sync();
    if (io.logits) store_logits(io.logits + ((size_t)s * T + t) * V, lg, V, lane);
    if (SCORE && !ROW && io.nll) {
        const int yv = scalar_load(io.targets + (size_t)s * T + t);
        if (yv >= 0 && yv < V) token_nll(nacc, lg, V, yv, lane);
        else if (lane == 0) atomicOr(m.err, 2u);
    }
    if (SCORE && io.digest) {
#pragma unroll
        for (int j = 0; j < L; j++) dg = dg * kDigestMul + sh.dterm[t % LG][j];
    }
}

// the update of token t by layer l (its record G arrived during the last ticks), its readout into the logits of token
// t, and the outputs; the last layer completes the token. It computes whether ok or not (the record is then read in
// every tick, so no path leaves its loads pending) and stores only for a token of the stream (ok).
// mid() runs once the update has read the record's A16, U' and table row (the single-buffer builds load the next
// record's there while the readout still reads P)
template <class SH, int L, int P, bool SCORE, bool GROUP, class Mid = NoHook>
__device__ __forceinline__ void flow_update(FlowShared<SH, L, P, GROUP, SCORE> &sh, const YggDevModel &m,
                                            const YggDevLayer &y, const Gather<SH> &G, const float (&bias)[4],
                                            int l, int t, bool ok, int r, int s, int T, const YggIO &io,
                                            unsigned long long &dg, NllSum &nacc, int lane, Mid mid = Mid()) {
    using F = SH;
    using FS = FlowShared<SH, L, P, GROUP, SCORE>;
    constexpr int QM = FS::QR - 1, LG = FS::LG;
    const int VP = m.VP;
    t = ok ? t : 0;
    int8_t *qnew = sh.qring[l][(t + 1) & QM];
    int qn[F::C];
    if (lane < F::NL) {
        const float *mul = nullptr;
        if constexpr (GROUP) mul = sh.GT.mul[l > 0 ? l - 1 : 0];
        const int *dpre = nullptr;
        if constexpr (FS::BIG) dpre = sh.dring[l][t & 1];
        update<SH, GROUP, FS::BIG>(qn, G, sh.qring[l][t & QM], sh.zlw[l][t & 3], y, l > 0, m.shift, lane, mul, dpre);
        if (ok) {
#pragma unroll
            for (int c = 0; c < F::C; c++) qnew[F::C * lane + c] = (int8_t)qn[c];
        }
    }
    mid();
    wave_sync();
    // (a token outside the stream reads out into the wave's own row, not the ring slot of a token in flight)
    int8_t *zq = (FS::ZQRING && ok) ? sh.zqr[FS::ZQRING ? l : 0][FS::ZQRING ? t % LG : 0] : sh.zqw[l];
    readout<SH>(zq, G.pw, qnew, GROUP ? G.mzr : y.readout_scale, lane);
    if constexpr (FS::LOGW) {
        // the logits wave adds the unembedding term after the barrier
        if (ok) flow_outputs<SH, L, P, SCORE, GROUP>(sh, m, qn, qnew, l, t, r, s, T, io, lane);
        return;
    }
    wave_sync();
    if (!ok) return;
    if constexpr (FS::ZQR) {
        flow_outputs<SH, L, P, SCORE, GROUP>(sh, m, qn, qnew, l, t, r, s, T, io, lane);
        if (l == L - 1) {
            // the logits of token t: the bias, then every layer's term in layer order
            float lg[4];
#pragma unroll
            for (int u = 0; u < 4; u++) lg[u] = bias[u];
#pragma unroll 1
            for (int j = 0; j < L; j++) {
                const YggDevLayer &yj = m.layers[j];
                float term[4];
                const float *sq = nullptr;
                if constexpr (GROUP) sq = sh.GT.sq[j];
                unembed_terms<SH::R, GROUP>(term, sh.zqr[FS::ZQR ? j : 0][FS::ZQR ? t % LG : 0], sh.S.Q[j],
                                            yj.unembed_scale, lane, sq);
#pragma unroll
                for (int u = 0; u < 4; u++) lg[u] = lg[u] + term[u];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? lg[u] : 0.0f;
            flow_finish<SH, L, P, SCORE, GROUP>(sh, m, lg, t, s, T, io, dg, nacc, lane);
        }
        return;
    }
    float *lr = sh.lgs[t % LG];
    if (4 * lane < VP) {
        float term[4];
        const float *sq = nullptr;
        if constexpr (GROUP) sq = sh.GT.sq[l];
        unembed_terms<SH::R, GROUP>(term, sh.zqw[l], sh.S.Q[l], y.unembed_scale, lane, sq);
#pragma unroll
        for (int u = 0; u < 4; u++) lr[4 * lane + u] = (l == 0 ? bias[u] : lr[4 * lane + u]) + term[u];
    }
    flow_outputs<SH, L, P, SCORE, GROUP>(sh, m, qn, qnew, l, t, r, s, T, io, lane);
    if (l == L - 1) {
        wave_sync();
        float lg[4];
#pragma unroll
        for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? lr[4 * lane + u] : 0.0f;
        flow_finish<SH, L, P, SCORE, GROUP>(sh, m, lg, t, s, T, io, dg, nacc, lane);
    }
}

// the NLL of token t, whose logits the last layer left in lgs[t & 1] last tick (the NLL wave)
template <class SH, int L, int P, bool GROUP>
__device__ __forceinline__ void flow_nll(FlowShared<SH, L, P, GROUP, true> &sh, const YggDevModel &m, int t, int s,
                                         int T, const YggIO &io, NllSum &nacc, int lane) {
    const int V = m.V, VP = m.VP;
    const float *lr = sh.lgs[t & 1];
    float lg[4];
#pragma unroll
    for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? lr[4 * lane + u] : 0.0f;
    const int yv = scalar_load(io.targets + (size_t)s * T + t);
    if (yv >= 0 && yv < V) token_nll(nacc, lg, V, yv, lane);
    else if (lane == 0) atomicOr(m.err, 2u);
}

// the logits of token t, a tick after the last layer's update (the logits wave): the bias, then every layer's
// unembedding term of the zq rows the layers left, in layer order (the reference's order of additions)
template <class SH, int L, int P, bool SCORE, bool GROUP>
__device__ __forceinline__ void flow_logits(FlowShared<SH, L, P, GROUP, SCORE> &sh, const YggDevModel &m,
                                            const float (&bias)[4], int t, int s, int T, const YggIO &io,
                                            unsigned long long &dg, NllSum &nacc, int lane) {
    using FS = FlowShared<SH, L, P, GROUP, SCORE>;
    float lg[4];
#pragma unroll
    for (int u = 0; u < 4; u++) lg[u] = bias[u];
#pragma unroll
    for (int j = 0; j < L; j++) {
        float term[4];
        const float *sq = nullptr;
        if constexpr (GROUP) sq = sh.GT.sq[j];
        unembed_terms<SH::R, GROUP>(term, sh.zqr[FS::ZQRING ? j : 0][FS::ZQRING ? t % FS::LG : 0], sh.S.Q[j],
                                    m.layers[j].unembed_scale, lane, sq);
#pragma unroll
        for (int u = 0; u < 4; u++) lg[u] = lg[u] + term[u];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < m.VP ? lg[u] : 0.0f;
    flow_finish<SH, L, P, SCORE, GROUP>(sh, m, lg, t, s, T, io, dg, nacc, lane);
}

// Wave w's role, 3 l + k: layer l's update wave (k = 0; the token layer's for l = 0) or a descent wave (k = 1; SPLIT:
// k = 1 and 2, of token parity 0 and 1); SPLIT: 2 the logits wave; LIW: 1 the layer-input wave. Wave w of a workgroup runs on SIMD w % 4, and the
// tables spread the work over the four: a layer's two descent waves, whose heavier set of rounds alternates tick by
// tick, share a SIMD where they can, and no two descent waves of the unsplit form do.
constexpr int kFlowLogitsRole = 2, kFlowLayerInputRole = 1;
template <int L, bool SPLIT> __device__ __forceinline__ int flow_role(int w) {
    if constexpr (SPLIT) {
        constexpr int r2[6] = {0, 3, 4, 5, 2, 1};
        constexpr int r3[8] = {0, 4, 7, 6, 3, 5, 8, 2};
        constexpr int r4[11] = {0, 3, 6, 9, 4, 7, 10, 11, 5, 8, 2};
        constexpr int r5[14] = {0, 6, 9, 12, 3, 7, 10, 13, 4, 8, 11, 14, 5, 2};
        return L == 2 ? r2[w] : L == 3 ? r3[w] : L == 4 ? r4[w] : r5[w];
    } else {
        constexpr int r4[7] = {0, 4, 3, 7, 10, 6, 9};
        constexpr int r5[9] = {0, 4, 7, 10, 3, 6, 9, 13, 12};
        if constexpr (L == 4) return r4[w];
        if constexpr (L == 5) return r5[w];
        return w == 0 ? 0 : 3 * ((w + 1) >> 1) + (w & 1);
    }
}

// MODE: kModeRun (logits, leaves, states) or kModeScore (also the digest and the NLL)
template <int N, int R, int R2, int L, int P, int MODE, bool GROUP>
__global__ __launch_bounds__((kFlowThreads<Shape<N, R, R2>, L, MODE>)) __attribute__((amdgpu_waves_per_eu(1)))
void flow_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                 const YggIO io) {
    using SH = Shape<N, R, R2>;
    using F = SH;
    constexpr bool SCORE = MODE == kModeScore, NLLW = kFlowNllWave<SH, L, MODE>;
    using FS = FlowShared<SH, L, P, GROUP, SCORE>;
    constexpr bool BIG = FS::BIG, VREG = FS::VREG;
    constexpr int QM = FS::QR - 1, NT = kFlowThreads<SH, L, MODE>;
    __shared__ __attribute__((aligned(16))) FS sh;

    // wave 0: the token layer; the routed layers' descent waves (SPLIT: two, for the tokens of parity dpar 0 and 1)
    // and update waves placed by flow_role; NLLW: the last wave the NLL; LOGW (the SPLIT builds): the logits wave
    // placed by flow_role (both set up as no layer's: descent set, layer 0)
    constexpr bool SPLIT = kFlowSplit<SH, L, MODE>, LOGW = FS::LOGW;
    static_assert(LOGW == SPLIT, "the split builds finish the logits on the logits wave");
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const bool nllw = NLLW && w == kFlowWaves<SH, L, MODE>;
    const int c = nllw ? 0 : flow_role<L, SPLIT>(w);
    constexpr bool LIW = kFlowLiw<SH, L, MODE>;
    // SB1 (the split builds of 4 layers or more with records of n = 128): one record buffer per update wave, reloaded
    // part by part as the update and the readout finish with it. About 25 fewer VGPRs: two resident workgroups per CU
    // instead of one (measured at 512-2048 streams: 5-16% faster). Where residency does not rise (fewer layers,
    // smaller records) the shorter load window cost up to 16%.
    constexpr bool SB1 = SPLIT && L >= 4 && N >= 128;
    const bool logw = LOGW && c == kFlowLogitsRole, liw = LIW && c == kFlowLayerInputRole;
    int l, dpar = 0;
    bool descent;
    if (nllw || logw || liw) {
        l = 0;
        descent = true;
    } else {
        l = c / 3;
        descent = c % 3 != 0;
        dpar = c % 3 == 2;
    }
    const int qk = lane & 3, qj = lane >> 2;
    const int s = blockIdx.x;
    const int V = m.V, VP = m.VP;
    load_tables<SH, L, NT, !VREG>(sh.S, m, tid);
    if constexpr (GROUP) load_group_tables<SH, L, NT>(sh.GT, m, tid);
    const YggDevLayer &y = m.layers[l];
    int8_t *st = state + ((size_t)s * L + l) * N;
    if (!descent) {
        for (int i = lane; i < N; i += 64) sh.qring[l][0][i] = st[i];     // the state before token 0
        if (lane < SH::ZL) {
#pragma unroll
            for (int j = 0; j < 4; j++) sh.zlw[l][j][lane] = 0;
        }
        if (lane < 4) sh.leafx[l][lane >> 1][lane & 1] = 0;
    }
    if (tid == 0) sh.stop_t = T;
    float bias[4];
#pragma unroll
    for (int u = 0; u < 4; u++) bias[u] = 4 * lane + u < VP ? m.output_bias[4 * lane + u] : 0.0f;
    __syncthreads();

    // (even: some waves run 2 a loop; NLLW, LOGW: one tick more each, for the NLL and the logits of the last token)
    const int ticks = (kFlowToken0 + (L - 1) * (P + 2) + T + 1 + (NLLW ? 1 : 0) + (LOGW ? 1 : 0)) & ~1;
    const int o_prev = kFlowToken0 + (l - 1) * (P + 2);                   // the layer below's update of token 0
    const int32_t *tok = tokens + (size_t)s * T;
    // the token at an index clamped into the stream (stages on tokens outside the stream or the vocabulary still run,
    // on token 0, and store nothing)
    auto token_at = [&](int t) { return scalar_load(tok + (t < 0 ? 0 : (t < T ? t : T - 1))); };
    // the wave that finishes the tokens: the logits wave, else the last layer's update wave
    const bool fin = LOGW ? logw : (l == L - 1 && !descent);
    unsigned long long dg = (SCORE && io.digest && fin) ? io.digest[s] : 0ull;
    NllSum nacc;
    // everything loaded so far has arrived: no value from before the ticks is waited for inside them
    __builtin_amdgcn_s_waitcnt(0);

    if (T > 0 && nllw) {
        // ---- the NLL wave: at tick k the NLL of the token whose logits were finished at tick k - 1, by the last
        // layer or (LOGW) the logits wave a tick after it (tokens from the stop on were not completed: the stop only
        // moves to a token the last layer has not reached)
        if constexpr (NLLW) {
            for (int k = 0; k < ticks; k++) {
                const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
                const int tn = k - 1 - kFlowToken0 - (L - 1) * (P + 2) - (LOGW ? 1 : 0);
                if (io.nll && tn >= 0 && tn < T && tn < stop) flow_nll<SH, L, P, GROUP>(sh, m, tn, s, T, io, nacc, lane);
                flow_barrier();
            }
        }
    } else if (T > 0 && liw) {
        // ---- the layer-input wave: at tick k the layer inputs of the tokens whose last router round ran at tick
        // k - 1, one per routed layer (their updates read them next tick; the state below is kept 8 tokens)
        if constexpr (LIW) {
            for (int k = 0; k < ticks; k++) {
                const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
#pragma unroll 1
                for (int li = 1; li < L; li++) {
                    const int t = k - kFlowToken0 - (li - 1) * (P + 2) - P - 1;
                    if (t >= 0 && t < T && t < stop) {
                        uint32_t qb[F::QW];
                        quad_share<N>(qb, sh.qring[li - 1][(t + 1) & QM], qk);
                        layer_input<SH>(sh.zlw[li][t & 3], sh.S.V[li - 1], sh.S.mv[li - 1], qb, sh.rhol[li][t & 3],
                                        lane);
                    }
                }
                flow_barrier();
            }
        }
    } else if (T > 0 && logw) {
        // ---- the logits wave: at tick k the logits of the token the last layer updated at tick k - 1 (tokens from
        // the stop on were not updated: the stop only moves to a token the last layer has not reached)
        if constexpr (LOGW) {
            for (int k = 0; k < ticks; k++) {
                const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
                const int tn = k - 1 - kFlowToken0 - (L - 1) * (P + 2);
                if (tn >= 0 && tn < T && tn < stop) flow_logits<SH, L, P, SCORE, GROUP>(sh, m, bias, tn, s, T, io, dg, nacc, lane);
                flow_barrier();
            }
        }
    } else if (T > 0 && l == 0) {
        // ---- the token layer: the record of token k at tick k into buffer k & 1, its update at tick k + 2 (before
        // that tick's record refills the buffer). SB1 (the split builds): one buffer, the record of token k - 1
        // loaded at tick k as the update of token k - 2 finishes with each part of the one before
        Gather<SH> G0, G1;
        int gx0 = 0, gx1 = 0;
        if constexpr (SB1) {
            for (int k = 0; k < ticks; k++) {
                const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
                const int xn = token_at(k - 1);
                const int t = k - kFlowToken0;
                bool ok = t >= 0 && t < T && t < stop;
                if (ok && (gx0 < 0 || gx0 >= V)) {
                    if (lane == 0) {
                        atomicOr(m.err, 1u);
                        sh.stop_t = t;
                    }
                    ok = false;
                }
                const int xg = (xn < 0 || xn >= V) ? 0 : xn;
                flow_update<SH, L, P, SCORE, GROUP>(sh, m, y, G0, bias, 0, t, ok, gx0, s, T, io, dg, nacc, lane,
                                                    [&]() { gather<SH, GROUP, true, false, 1>(G0, y, xg, xg, false, lane); });
                gather<SH, GROUP, true, false, 2>(G0, y, xg, xg, false, lane);
                gx0 = xn;
                flow_barrier();
            }
        }
        auto tick = [&](int k, Gather<SH> &G, int &gx) {
            const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
            const int xn = token_at(k);
            const int t = k - kFlowToken0;
            bool ok = t >= 0 && t < T && t < stop;
            if (ok && (gx < 0 || gx >= V)) {
                if (lane == 0) {
                    atomicOr(m.err, 1u);
                    sh.stop_t = t;
                }
                ok = false;
            }
            flow_update<SH, L, P, SCORE, GROUP>(sh, m, y, G, bias, 0, t, ok, gx, s, T, io, dg, nacc, lane);
            gx = xn;
            const int xg = (xn < 0 || xn >= V) ? 0 : xn;
            gather<SH, GROUP>(G, y, xg, xg, false, lane);
            flow_barrier();
        };
        if constexpr (!SB1) {
            for (int k = 0; k < ticks; k += 2) {
                tick(k, G0, gx0);
                tick(k + 1, G1, gx1);
            }
        }
    } else if (T > 0 && !descent) {
        // ---- a routed layer's update wave: at tick k the record of token k - o_prev - P - 1 (its leaf left by the
        // descent wave last tick) into buffer k & 1, then the update of the token before it from the other buffer
        const int o_g = o_prev + P + 1;
        Gather<SH> G0, G1;
        int gr0 = 0, gr1 = 0;
        if constexpr (SB1) {
            // (one buffer: the update of token k - o_g - 1 from the record loaded last tick, and as it finishes with
            // each part of it, that part of the record of token k - o_g)
            for (int k = 0; k < ticks; k++) {
                const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
                const int tg = k - o_g;
                const int *lx = sh.leafx[l][tg & 1];
                const int r = __builtin_amdgcn_readfirstlane(lx[0]), x = __builtin_amdgcn_readfirstlane(lx[1]);
                const int t = tg - 1;
                flow_update<SH, L, P, SCORE, GROUP>(sh, m, y, G0, bias, l, t, t >= 0 && t < T && t < stop, gr0, s, T,
                                                    io, dg, nacc, lane,
                                                    [&]() { gather<SH, GROUP, !BIG, false, 1>(G0, y, r, x, true, lane); });
                gather<SH, GROUP, !BIG, false, 2>(G0, y, r, x, true, lane);
                gr0 = r;
                flow_barrier();
            }
        }
        auto tick = [&](int k, Gather<SH> &Gg, int &grg, const Gather<SH> &Gu, int gru) {
            const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
            const int tg = k - o_g;
            const int *lx = sh.leafx[l][tg & 1];
            const int r = __builtin_amdgcn_readfirstlane(lx[0]), x = __builtin_amdgcn_readfirstlane(lx[1]);
            grg = r;
            gather<SH, GROUP, !BIG>(Gg, y, r, x, true, lane);
            const int t = tg - 1;
            flow_update<SH, L, P, SCORE, GROUP>(sh, m, y, Gu, bias, l, t, t >= 0 && t < T && t < stop, gru, s, T, io,
                                                dg, nacc, lane);
            flow_barrier();
        };
        if constexpr (!SB1) {
            for (int k = 0; k < ticks; k += 2) {
                tick(k, G0, gr0, G1, gr1);
                tick(k + 1, G1, gr1, G0, gr0);
            }
        }
    } else if (T > 0) {
        // ---- a descent wave: its router plan (round j: rh[j] levels from slot rb[j], subtrees at depth rd[j])
        int rh[P], rb[P], rd[P];
        {
            int base = 1 << m.round_h[0], d0 = m.round_h[0];
            rh[0] = m.round_h[0];
            rb[0] = 0;
            rd[0] = 0;
#pragma unroll
            for (int j = 1; j < P; j++) {
                rh[j] = (m.round_pack >> (4 * j)) & 15;
                rb[j] = base;
                rd[j] = d0;
                base += (1 << d0) << rh[j];
                d0 += rh[j];
            }
        }
        const int nn0 = (1 << rh[0]) - 1;
        const int8_t *w0 = sh.S.W[l - 1] + (qj < nn0 ? qj : nn0 - 1) * kLdsRow<N>;
        // BIG: V' in registers, and the U' share of the last leaf reached (its products with zl next tick)
        uint32_t vr[VREG ? SH::RG : 1][F::QW];
        uint32_t uwp[BIG ? SH::K4 : 1][F::C];
        if constexpr (BIG) {
            if constexpr (VREG) load_vrows<SH>(vr, y, lane);
#pragma unroll
            for (int k4 = 0; k4 < SH::K4; k4++)
#pragma unroll
                for (int c = 0; c < F::C; c++) uwp[k4][c] = 0u;
            __builtin_amdgcn_s_waitcnt(0);
        }
        // carried from tick to tick: each pending round's row shares, threshold, node, rho and token (round j's
        // inputs, loaded by round j - 1; th[0] the first round's thresholds)
        uint32_t wv[P][F::QW];
        float th[P], rhos[P];
        int ixs[P], xs[P];
#pragma unroll
        for (int j = 0; j < P; j++) {
            th[j] = 0.0f;
            rhos[j] = 0.0f;
            ixs[j] = 1 << rd[j];
            xs[j] = 0;
#pragma unroll
            for (int i = 0; i < F::QW; i++) wv[j][i] = 0u;
        }
        // one tick: A < 0 every round, else (SPLIT) the rounds j with j % 2 == A (the rest are the other wave's)
        auto dtick = [&](int k, auto A_) {
            constexpr int A = decltype(A_)::value;
            const int stop = __builtin_amdgcn_readfirstlane(sh.stop_t);
            const int t0 = k - o_prev;                            // the token whose first-round thresholds load now
            const int xr = token_at(t0);
            // ---- router rounds, the last first (each consumes what the one before it loaded last tick)
            int lx = 0, lr = 0, lt = 0;
            float lrho = 0.0f;
#pragma unroll
            for (int j = P - 1; j >= 0; j--) {
                if (A >= 0 && (j & 1) != A) continue;          // (SPLIT: the other wave's round this tick)
                const int t = k - o_prev - 1 - j;
                uint32_t qbw[F::QW];
                int ix, x;
                float rho;
                if (j == 0) {
                    x = xs[0];
                    rho = below_and_rho<N>(qbw, sh.qring[l - 1][(t + 1) & QM], y.rms_eps, lane);
                    if constexpr (GROUP)
                        if (y.r2b) rho = group_rho<N>(qbw, sh.GT.r2[l - 1], y.rms_eps);
                    uint32_t wr[F::QW];
                    quad_share<N>(wr, w0, qk);
                    ix = round_step<N>(wr, qbw, rho, th[0], 1, rh[0], lane);
                } else {
                    x = xs[j];
                    rho = rhos[j];
                    quad_share<N>(qbw, sh.qring[l - 1][(t + 1) & QM], qk);
                    ix = round_step<N>(wv[j], qbw, rho, th[j], ixs[j], rh[j], lane);
                }
                if (j + 1 < P) {
                    // the next round's row shares and thresholds, for next tick (quads past the round's nodes
                    // read its last node's row: no extra cache line)
                    const int jn = j + 1 < P ? j + 1 : P - 1;     // (constant once unrolled)
                    const int nn = (1 << rh[jn]) - 1;
                    const int slot = rb[jn] + ((ix - (1 << rd[jn])) << rh[jn]) + (qj < nn ? qj : nn - 1);
                    quad_share<N>(wv[jn], y.w + (size_t)slot * N, qk);
                    th[jn] = y.thr[(size_t)x * y.thr_stride + slot];
                    ixs[jn] = ix;
                    rhos[jn] = rho;
                    xs[jn] = x;
                } else {
                    lt = t;
                    lx = x;
                    lr = ix - m.E;
                    lrho = rho;
                    // ---- the leaf reached and its layer input, for the update wave: before the earlier rounds, whose
                    // inputs were loaded later last tick and are still arriving (LIW: the rho, for the layer-input
                    // wave next tick)
                    if (lt >= 0 && lt < T && lt < stop) {
                        if (lane == 0) {
                            sh.leafx[l][lt & 1][0] = lr;
                            sh.leafx[l][lt & 1][1] = lx;
                            if constexpr (LIW) sh.rhol[l][lt & 3] = lrho;
                        }
                    }
                    if (!LIW && lt >= 0 && lt < T && lt < stop) {
                        uint32_t qb[F::QW];
                        quad_share<N>(qb, sh.qring[l - 1][(lt + 1) & QM], qk);
                        if constexpr (VREG)
                            layer_input_regs<SH>(sh.zlw[l][lt & 3], vr, sh.S.mv[l - 1], qb, lrho, lane);
                        else
                            layer_input<SH>(sh.zlw[l][lt & 3], sh.S.V[l - 1], sh.S.mv[l - 1], qb, lrho, lane);
                    }
                }
            }
            if constexpr (BIG) {
                // ---- the U'z products of the leaf before (its U' arrived during this tick), for the update wave's
                // next tick; then the U' of the leaf just reached
                const int tu = lt - 1;
                int d[F::C];
                uw_products<SH>(d, uwp, sh.zlw[l][tu & 3]);
                if (tu >= 0 && tu < T && tu < stop && lane < F::NL) {
#pragma unroll
                    for (int c = 0; c < F::C; c++) sh.dring[l][tu & 1][F::C * lane + c] = d[c];
                }
                load_uw<SH>(uwp, y, lr, lane);
            }
            // ---- the first round's thresholds of token t0, for next tick (SPLIT: by the wave whose round 0 it is)
            if (A < 0 || A == 1) {
                const int x0 = (xr < 0 || xr >= V) ? 0 : xr;
                th[0] = y.thr[(size_t)x0 * y.thr_stride + (qj < nn0 ? qj : nn0 - 1)];
                xs[0] = x0;
            }
            flow_barrier();
        };
        if constexpr (SPLIT) {
            // round j of token t runs in tick o_prev + 1 + t + j, so this wave's rounds in tick k are those with
            // j = k + o_prev + 1 + dpar (mod 2): in even ticks those of parity a0
            const int a0 = (o_prev + 1 + dpar) & 1;
            if (a0 == 0) {
                for (int k = 0; k < ticks; k += 2) {
                    dtick(k, std::integral_constant<int, 0>());
                    dtick(k + 1, std::integral_constant<int, 1>());
                }
            } else {
                for (int k = 0; k < ticks; k += 2) {
                    dtick(k, std::integral_constant<int, 1>());
                    dtick(k + 1, std::integral_constant<int, 0>());
                }
            }
        } else {
            for (int k = 0; k < ticks; k++) dtick(k, std::integral_constant<int, -1>());
        }
    }
    __syncthreads();
    if (!descent) {
        const int te = T < sh.stop_t ? T : sh.stop_t;                // tokens processed
        for (int i = lane; i < N; i += 64) st[i] = sh.qring[l][te & QM][i];
    }
    if (SCORE && io.digest && fin && lane == 0) io.digest[s] = dg;
    if (SCORE && io.nll && (NLLW ? nllw : fin) && lane == 0) io.nll[s] += nacc.value();
}

}  // namespace ygg
