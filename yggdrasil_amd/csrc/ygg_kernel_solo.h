// solo_kernel: one stream per workgroup with all four wavefronts working on it, for calls of few streams whose tokens
// wait on each other (a one-token ygg_step captured in a graph, ygg_generate). Same arithmetic and lane mappings as
// fast_kernel (ygg_kernel_fast.h), whose per-layer pieces it reuses.
//
// What makes a token's chain short:
//   - nothing is staged before the first token but Q, V' and the layer-input scales (small, in LDS), and every load
//     that does not depend on the stream's data is issued at entry: the state, the first token and, in registers,
//     each routed layer's router rows of the first two rounds of its plan ("round A", up to 8 levels, 255 nodes:
//     lane i of the workgroup holds node i's whole row);
//   - round A is one step of arithmetic: every lane forms its node's comparison (f32(w . q) rho > thr[x][node]) and
//     the four wavefronts' ballots, combined in LDS, give wavefront 0 the path through all its levels;
//   - the rounds after it (at most 6 levels, at most 63 nodes) are one round with one lane of wavefront 0 per node,
//     as in fast_kernel's deep descent;
//   - so a routed layer costs two dependent global loads (that round's rows, then the leaf's record), and the
//     token layer one (its record) after the token.
// Work split per routed layer l: all wavefronts form round A's comparisons (one workgroup barrier hands the ballots to
// wavefront 0); wavefront 0 walks the path, issues the last round's loads, forms the layer input zl (V' . q_below)
// while they are on the way, finishes the descent, gathers the record, updates the state, reads it out and adds the
// layer's unembedding term to the logits (in layer order, the reference's order, cpu/ygg.cpp:457); a second barrier
// hands the new state to every wavefront for the next layer's round A. After the last layer wavefront 0 stores the
// logits and, when generating, samples the next token.
//
// Router plans it takes: 1 to 4 rounds, the first two at most 8 levels together, the third and fourth at most 6
// (every depth up to 14 in the default plan). Round A's rows take (L - 1) n / 4 registers per lane, so (L - 1) n is
// at most 512.
#pragma once
#include "ygg_kernel_fast.h"

namespace ygg {

constexpr int kSoloThreads = 256;

template <int N, int L> constexpr bool kSoloRowsFit = (L - 1) * N <= 512;

// LDS of a solo workgroup: the unembedding Q of every layer (in the planes of SharedTables), V' and m_v of every
// routed layer, the states, the layer input, every layer's readout of the current token, round A's ballots
template <class SH, int L> struct SoloShared {
    static constexpr int LR = L > 1 ? L - 1 : 1;
    alignas(16) int8_t Q[L][256 * SH::R];
    alignas(16) int8_t V[LR][SH::R2 * kLdsRow<SH::N>];
    alignas(16) float mv[LR][SH::R2];
    alignas(16) int8_t qs[L][SH::N];
    alignas(16) int8_t zl[SH::ZL];
    alignas(16) int8_t zq[L][SH::ZQ];
    unsigned long long masks[4];
    int next_x;
    // where threads with nothing to stage store at entry (no store is conditional: see solo_tables_store)
    alignas(16) uint4 sink[kSoloThreads];
};

// Q, V' and m_v into LDS by all threads (the layout of load_tables): the loads into registers first (solo_tables_load),
// the LDS stores later (solo_tables_store), so that loads issued in between stay in flight past the stores' waits
template <class SH, int L> struct SoloStage {
    static constexpr int LR = L > 1 ? L - 1 : 1, NT = kSoloThreads;
    static constexpr int QK = (16 * SH::R + NT - 1) / NT;
    static constexpr int VK = (SH::R2 * (SH::N / 16) + NT - 1) / NT;
    uint4 qv[L][QK], vv[LR][VK];
    float mvv[LR];
};

template <class SH, int L>
__device__ __forceinline__ void solo_tables_load(SoloStage<SH, L> &G, const YggDevModel &m, int tid) {
    using ST = SoloStage<SH, L>;
    constexpr int R2 = SH::R2, RC = SH::N / 16, NT = ST::NT;
    static_assert(NT >= R2, "one thread per m_v entry");
    // (every load is issued by every thread, at an index clamped into the array: with no branch around a load the
    // compiler counts the loads in flight and later waits wait for the ones they need, not for all of them; the
    // stores skip the clamped entries)
    const int qch = m.VP * SH::R / 16;
#pragma unroll
    for (int l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < ST::QK; k++) {
            const int c = tid + k * NT;
            G.qv[l][k] = ((const uint4 *)m.layers[l].Q)[c < qch ? c : 0];
        }
#pragma unroll
    for (int l = 1; l < L; l++)
#pragma unroll
        for (int k = 0; k < ST::VK; k++) {
            const int c = tid + k * NT;
            G.vv[l - 1][k] = ((const uint4 *)m.layers[l].vl)[c < R2 * RC ? c : 0];
        }
    // (every layer's m_v by threads tid < R2, each load through the layer's uniform pointer: a per-thread choice of
    // layer would read the pointer itself from the kernel argument with a vector load)
#pragma unroll
    for (int l = 1; l < L; l++) G.mvv[l - 1] = m.layers[l].mv[tid < R2 ? tid : 0];
}

// (every store is unconditional, threads past an array's end writing to S.sink: a store under a branch lets the
// compiler move its load into the branch, behind later loads, and wait for all of them there)
template <class SH, int L>
__device__ __forceinline__ void solo_tables_store(SoloShared<SH, L> &S, const SoloStage<SH, L> &G, const YggDevModel &m,
                                                  int tid) {
    using ST = SoloStage<SH, L>;
    constexpr int R2 = SH::R2, QC = SH::QC, RC = SH::N / 16, SC = kLdsRow<SH::N> / 16, NT = ST::NT;
    const int qch = m.VP * SH::R / 16;
#pragma unroll
    for (int l = 0; l < L; l++)
#pragma unroll
        for (int k = 0; k < ST::QK; k++) {
            const int c = tid + k * NT;
            uint4 *d = c < qch ? (uint4 *)S.Q[l] + (c % QC) * 64 + c / QC : S.sink + tid;
            *d = G.qv[l][k];
        }
#pragma unroll
    for (int l = 1; l < L; l++)
#pragma unroll
        for (int k = 0; k < ST::VK; k++) {
            const int c = tid + k * NT;
            uint4 *d = c < R2 * RC ? (uint4 *)S.V[l - 1] + (c / RC) * SC + c % RC : S.sink + tid;
            *d = G.vv[l - 1][k];
        }
#pragma unroll
    for (int l = 1; l < L; l++) {
        float *d = tid < R2 ? &S.mv[l - 1][tid] : (float *)(S.sink + tid);
        *d = G.mvv[l - 1];
    }
}

// Round A of the plan: its first two rounds, h0 + h1 <= 8 levels (h1 = 0 for a one-round plan). Thread tid takes
// one node: tid < 2^h0 - 1 the first round's nodes (slot tid), the next 2^h0 (2^h1 - 1) threads the second round's
// blocks one after the other (block c, node p: slot 2^h0 + c 2^h1 + p). slot -1: no node.
struct RoundA {
    int h0, h1, nn0, nn1, slot;
};
__device__ __forceinline__ RoundA round_a(const YggDevModel &m, int tid) {
    RoundA a;
    a.h0 = m.round_h[0];
    a.h1 = m.n_rounds > 1 ? m.round_h[1] : 0;
    a.nn0 = (1 << a.h0) - 1;
    a.nn1 = (1 << a.h1) - 1;
    a.slot = -1;
    if (tid < a.nn0) {
        a.slot = tid;
    } else if (a.nn1 > 0 && tid < a.nn0 + (a.nn1 << a.h0)) {
        const int j = tid - a.nn0, c = j / a.nn1;
        a.slot = (1 << a.h0) + (c << a.h1) + (j - c * a.nn1);
    }
    return a;
}

// bits [o, o + 32) of the workgroup's 256-bit ballot (o < 256)
__device__ __forceinline__ unsigned long long mask_bits(const unsigned long long (&mk)[4], int o) {
    const int w = o >> 6, b = o & 63;
    unsigned long long v = mk[w & 3] >> b;
    if (b && w < 3) v |= mk[w + 1] << (64 - b);
    return v;
}

// round A's path from the four ballots (thread tid's bit at bit tid) -> the node reached (heap index) at depth h0 + h1
__device__ __forceinline__ int walk_a(const unsigned long long (&mk)[4], const RoundA &a) {
    const int c0 = walk_bits(mk[0], a.h0) - a.nn0;
    int ix = (1 << a.h0) + c0;
    if (a.h1 > 0) {
        const int c1 = walk_bits(mask_bits(mk, a.nn0 + c0 * a.nn1), a.h1) - a.nn1;
        ix = (ix << a.h1) + c1;
    }
    return ix;
}

// walk h <= 4 levels of a subtree whose node j (breadth-first) goes right when bit (j << S) of mask is set -> the node
// index reached, in [2^h - 1, 2^(h+1) - 2] (wavefront-uniform, scalar)
__device__ __forceinline__ int walk_strided(unsigned long long mask, int h, int S) {
    int j = 0;
    for (int k = 0; k < h; k++) j = 2 * j + 1 + (int)((mask >> (j << S)) & 1ull);
    return j;
}

// The last round coalesced (n of 64, 128 or 256): its rows lie in two contiguous runs of slots, the third round's block
// of 2^h2 rows below ix and the 2^h2 fourth-round blocks below that (2^(h2 + h3) rows). Each load instruction reads
// 1 KiB of them (lane i: 16-byte chunk i % CR of a row, CR = n / 16 chunks per row, 64 / CR rows per instruction), the
// CR lanes of a row sum their partial dot products, and the first lane of a row compares. Row r of a run has its
// decision at bit (r CR) % 64 of the ballot of instruction (r CR) / 64 of that run. Needs 2^h2 CR <= 64 and
// 2^h3 CR <= 64 (kTailCoOk), so that a walked block lies in one ballot.
template <int N> constexpr int kTailCR = N / 16;
template <int N> constexpr bool kTailCo = N == 64 || N == 128 || N == 256;
__device__ __forceinline__ bool tail_co_ok(const YggDevModel &m, int cr) {
    if (m.n_rounds < 3) return false;
    if ((1 << m.round_h[2]) * cr > 64) return false;
    return m.n_rounds < 4 || (1 << m.round_h[3]) * cr <= 64;
}
template <int N>
__device__ __forceinline__ int tail_coalesced(const YggDevModel &m, const YggDevLayer &y, int ix, int d01, int x,
                                              const int8_t *qb, float rho, int lane) {
    constexpr int CR = kTailCR<N>, SH = CR == 4 ? 2 : (CR == 8 ? 3 : 4), MAXI = 1 + CR;
    const int h0 = m.round_h[0], h1 = m.round_h[1], h2 = m.round_h[2], h3 = m.n_rounds > 3 ? m.round_h[3] : 0;
    const int sub = ix - (1 << d01);
    const int base2 = (1 << h0) + (1 << (h0 + h1)), base3 = base2 + (1 << (d01 + h2));
    const int rb1 = base2 + (sub << h2), nr1 = 1 << h2;                 // first run: slots, rows
    const int rb2 = base3 + (sub << (h2 + h3)), nr2 = h3 ? 1 << (h2 + h3) : 0;
    const int i1 = (nr1 * CR + 63) >> 6, ni = i1 + ((nr2 * CR) >> 6);    // instructions
    // this lane's 16 bytes of the state below (chunk lane % CR of every row)
    uint32_t qc[4];
    load_words<4, 16>(qc, qb + (lane % CR) * 16);
    const float *thr = y.thr + (size_t)x * y.thr_stride;
    uint4 v[MAXI];
    float th[MAXI];
    // (every instruction loads, at a row clamped into its run: no branch around the loads, see solo_tables_load;
    // the clamped rows' decisions are masked below)
#pragma unroll
    for (int j = 0; j < MAXI; j++) {
        const int jj = j < ni ? j : 0;
        const int jr = jj < i1 ? jj : jj - i1, rb = jj < i1 ? rb1 : rb2, nr = jj < i1 ? nr1 : nr2;
        const int row = (64 * jr + lane) / CR, rowc = row < nr ? row : nr - 1;
        v[j] = *(const uint4 *)(y.w + ((size_t)rb + rowc) * N + (size_t)((lane % CR) * 16));
        th[j] = thr[rb + rowc];
    }
    unsigned long long bm[MAXI];
#pragma unroll
    for (int j = 0; j < MAXI; j++) {
        int p = dot4(v[j].x, qc[0], 0);
        p = dot4(v[j].y, qc[1], p);
        p = dot4(v[j].z, qc[2], p);
        p = dot4(v[j].w, qc[3], p);
        if constexpr (CR == 4) {
            p = sum4(p);
        } else if constexpr (CR == 8) {
            p = sum8(p);
        } else {
            p = sum8(p);
            p = p + __builtin_amdgcn_update_dpp(0, p, 0x140, 0xF, 0xF, false);   // row_mirror: the 16-lane sum
        }
        const int jr = j < i1 ? j : j - i1, nr = j < i1 ? nr1 : nr2;
        bm[j] = lane_mask(j < ni && (64 * jr + lane) / CR < nr && lane % CR == 0 && (float)p * rho > th[j]);
    }
    const int nn2 = (1 << h2) - 1;
    const int c = walk_strided(bm[0], h2, SH) - nn2;
    ix = (ix << h2) + c;
    if (h3) {
        const int nn3 = (1 << h3) - 1;
        const int bit = (c << h3) * CR, jb = i1 + (bit >> 6);
        unsigned long long mk = bm[0];
#pragma unroll
        for (int j = 1; j < MAXI; j++) mk = j == jb ? bm[j] : mk;
        ix = (ix << h3) + (walk_strided(mk >> (bit & 63), h3, SH) - nn3);
    }
    return ix;
}

// n-byte state row at qb (LDS) as dwords
template <int N> __device__ __forceinline__ void full_row(uint32_t (&q)[N / 4], const int8_t *qb) {
    load_words<N / 4, 16>(q, qb);
}

// MODE: kModeRun (logits, leaves, states after every token) or kModeGenerate (io.gen: the token sampled after every
// step is the next input). GROUP: the model has group scales.
template <int N, int R, int R2, int L, int MODE, bool GROUP>
__global__ __launch_bounds__(kSoloThreads) __attribute__((amdgpu_waves_per_eu(1)))
void solo_kernel(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T, int8_t *__restrict__ state,
                 const YggIO io) {
    using SH = Shape<N, R, R2>;
    using F = SH;
    constexpr int LR = L > 1 ? L - 1 : 1, NW = N / 4;
    constexpr bool GEN = MODE == kModeGenerate;
    static_assert(L >= 2 && kSoloRowsFit<N, L>, "solo_kernel: routed layers whose round-A rows fit registers");
    __shared__ __attribute__((aligned(16))) SoloShared<SH, L> S;
    __shared__ __attribute__((aligned(16))) GroupTablesOf<SH, L, GROUP> GT;

    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int s = blockIdx.x;
    const int V = m.V, VP = m.VP;
    touch_args<L>(m);
    // entry: the first token and the state, the LDS tables' loads, then round A's rows (registers, not waited for
    // until layer 1 of the first token), then the tables' stores
    const int32_t *tok = tokens + (size_t)s * (GEN ? 1 : T);
    int x_next = T > 0 ? __builtin_amdgcn_readfirstlane(tok[0]) : 0;
    int8_t *st = state + (size_t)s * L * N;
    constexpr int SB = (L * N + kSoloThreads - 1) / kSoloThreads;
    int sb[SB];
#pragma unroll
    for (int k = 0; k < SB; k++) sb[k] = st[tid + kSoloThreads * k < L * N ? tid + kSoloThreads * k : 0];
    SoloStage<SH, L> stage;
    solo_tables_load<SH, L>(stage, m, tid);
    const RoundA ra = round_a(m, tid);
    uint32_t rowa[LR][NW];
    const int slot_a = ra.slot >= 0 ? ra.slot : 0;       // (threads without a node load node 1's row, unused)
#pragma unroll
    for (int l = 1; l < L; l++) load_words<NW, 16>(rowa[l - 1], m.layers[l].w + (size_t)slot_a * N);
    solo_tables_store<SH, L>(S, stage, m, tid);
    if constexpr (GROUP) load_group_tables<SH, L, kSoloThreads>(GT, m, tid);
#pragma unroll
    for (int k = 0; k < SB; k++) {
        int8_t *d = tid + kSoloThreads * k < L * N ? &S.qs[0][tid + kSoloThreads * k] : (int8_t *)(S.sink + tid);
        *d = (int8_t)sb[k];
    }
    if (tid < SH::ZL) S.zl[tid] = 0;
    const Tail tl = make_tail(m, lane);
    __syncthreads();

    for (int t = 0; t < T; t++) {
        const int x = x_next;
        if (x < 0 || x >= V) {
            if (tid == 0) atomicOr(m.err, 1u);
            break;
        }
        if (!GEN && t + 1 < T) x_next = __builtin_amdgcn_readfirstlane(tok[t + 1]);
        // ---- the token layer (wavefront 0): its record as soon as the token is known, every thread's round-A
        // thresholds of every routed layer behind it; the layer's unembedding term starts the logits
        Gather<SH> G;
        if (wv == 0) gather<SH, GROUP>(G, m.layers[0], x, x, false, lane);
        float tha[LR];
#pragma unroll
        for (int l = 1; l < L; l++)
            tha[l - 1] = m.layers[l].thr[(size_t)x * m.layers[l].thr_stride + slot_a];
        float lg[4];
        if (wv == 0) {
            int qn[F::C];
            const YggDevLayer &y0 = m.layers[0];
            if (lane < F::NL) update<SH, GROUP>(qn, G, S.qs[0], S.zl, y0, false, m.shift, lane);
            wave_sync();
            if (lane < F::NL) {
#pragma unroll
                for (int c = 0; c < F::C; c++) S.qs[0][F::C * lane + c] = (int8_t)qn[c];
            }
            wave_sync();
            readout<SH>(S.zq[0], G.pw, S.qs[0], GROUP ? G.mzr : y0.readout_scale, lane);
            if (io.leaves && lane == 0) io.leaves[((size_t)s * T + t) * L] = x;
            wave_sync();
#pragma unroll
            for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? m.output_bias[4 * lane + u] : 0.0f;
            if (4 * lane < VP) {
                float term[4];
                const float *sq = nullptr;
                if constexpr (GROUP) sq = GT.sq[0];
                unembed_terms<R, GROUP>(term, S.zq[0], S.Q[0], y0.unembed_scale, lane, sq);
#pragma unroll
                for (int u = 0; u < 4; u++) lg[u] = lg[u] + term[u];
            }
        }
        __syncthreads();

        // ---- routed layers: round A on every wavefront, the rest of the layer on wavefront 0
#pragma unroll 1
        for (int l = 1; l < L; l++) {
            const YggDevLayer &y = m.layers[l];
            const int8_t *qb = S.qs[l - 1];
            uint32_t qbw[F::QW];
            float rho = below_and_rho<N>(qbw, qb, y.rms_eps, lane);
            if constexpr (GROUP)
                if (y.r2b) rho = group_rho<N>(qbw, GT.r2[l - 1], y.rms_eps);
            float th = tha[0];
#pragma unroll
            for (int i = 1; i < LR; i++) th = l - 1 == i ? tha[i] : th;
            uint32_t qf[NW];
            full_row<N>(qf, qb);
            // (four independent chains: with one wavefront per SIMD nothing hides a chain's latency)
            int dp[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < NW; i++) {
                uint32_t wsel = rowa[0][i];
#pragma unroll
                for (int k = 1; k < LR; k++) wsel = l - 1 == k ? rowa[k][i] : wsel;
                dp[i & 3] = dot4(wsel, qf[i], dp[i & 3]);
            }
            const int dot = (dp[0] + dp[1]) + (dp[2] + dp[3]);
            const unsigned long long bm = lane_mask(ra.slot >= 0 && (float)dot * rho > th);
            if (lane == 0) S.masks[wv] = bm;
            __syncthreads();
            if (wv == 0) {
                unsigned long long mk[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const unsigned long long v = S.masks[k];
                    mk[k] = ((unsigned long long)__builtin_amdgcn_readfirstlane((unsigned)(v >> 32)) << 32) |
                            (unsigned)__builtin_amdgcn_readfirstlane((unsigned)v);
                }
                int ix = walk_a(mk, ra);
                bool co = false;
                if constexpr (kTailCo<N>) co = tail_co_ok(m, kTailCR<N>);
                if (co) {
                    // the last round, coalesced; the layer input is formed after it (its rows' loads are waited
                    // for inside)
                    ix = tail_coalesced<N>(m, y, ix, ra.h0 + ra.h1, x, qb, rho, lane);
                    layer_input<SH>(S.zl, S.V[l - 1], S.mv[l - 1], qbw, rho, lane);
                } else if (m.n_rounds > 2) {
                    // the last round (the plan's third and fourth rounds): the nodes below ix, one lane each; the
                    // layer input is formed while their rows are on the way
                    const float *thr = y.thr + (size_t)x * y.thr_stride;
                    const int slot = tl.ta + ((ix - (1 << (ra.h0 + ra.h1))) << tl.tsh);
                    // (lanes off the round load its first row, unused: no branch around the loads)
                    const int slot_t = tl.on ? slot : tl.ta;
                    uint32_t tw[NW];
                    load_words<NW, 16>(tw, y.w + (size_t)slot_t * N);
                    const float tth = thr[slot_t];
                    layer_input<SH>(S.zl, S.V[l - 1], S.mv[l - 1], qbw, rho, lane);
                    uint32_t qt[NW];                  // (read again: round A's copy need not stay live)
                    full_row<N>(qt, qb);
                    int tq[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int i = 0; i < NW; i++) tq[i & 3] = dot4(tw[i], qt[i], tq[i & 3]);
                    const int td = (tq[0] + tq[1]) + (tq[2] + tq[3]);
                    const unsigned long long mask = lane_mask(tl.on && (float)td * rho > tth);
                    const int h2 = m.round_h[2], nn2 = (1 << h2) - 1;
                    const int c = walk_bits(mask, h2) - nn2;
                    ix = (ix << h2) + c;
                    if (m.n_rounds == 4) {
                        const int h3 = m.round_h[3], nn3 = (1 << h3) - 1;
                        ix = (ix << h3) + (walk_bits(mask >> (nn2 + c * nn3), h3) - nn3);
                    }
                } else {
                    layer_input<SH>(S.zl, S.V[l - 1], S.mv[l - 1], qbw, rho, lane);
                }
                const int r = ix - m.E;
                gather<SH, GROUP>(G, y, r, x, true, lane);
                if (io.leaves && lane == 0) io.leaves[((size_t)s * T + t) * L + l] = r;
                wave_sync();
                int qn[F::C];
                const float *mul = nullptr;
                if constexpr (GROUP) mul = GT.mul[l - 1];
                if (lane < F::NL) update<SH, GROUP>(qn, G, S.qs[l], S.zl, y, true, m.shift, lane, mul);
                wave_sync();
                if (lane < F::NL) {
#pragma unroll
                    for (int c = 0; c < F::C; c++) S.qs[l][F::C * lane + c] = (int8_t)qn[c];
                }
                wave_sync();
                readout<SH>(S.zq[l], G.pw, S.qs[l], GROUP ? G.mzr : y.readout_scale, lane);
                wave_sync();
                if (4 * lane < VP) {
                    float term[4];
                    const float *sq = nullptr;
                    if constexpr (GROUP) sq = GT.sq[l];
                    unembed_terms<R, GROUP>(term, S.zq[l], S.Q[l], y.unembed_scale, lane, sq);
#pragma unroll
                    for (int u = 0; u < 4; u++) lg[u] = lg[u] + term[u];
                }
                if (l == L - 1) {
                    // the token is complete: logits, states, and the next token when generating
                    if (io.logits) store_logits(io.logits + ((size_t)s * T + t) * V, lg, V, lane);
                    if (io.states) {
                        int8_t *so = io.states + ((size_t)s * T + t) * L * N;
                        for (int i = lane; i < L * N; i += 64) so[i] = S.qs[0][i];
                    }
                    if constexpr (GEN) {
                        const int nx = sample_token(lg, V, io.temperature, io.top_k, io.seed, s, t, lane);
                        if (lane == 0) {
                            io.gen[(size_t)s * T + t] = nx;
                            S.next_x = nx;
                        }
                    }
                }
            }
            __syncthreads();
        }
        if constexpr (GEN) x_next = __builtin_amdgcn_readfirstlane(S.next_x);
    }
    __syncthreads();
    for (int i = tid; i < L * N; i += kSoloThreads) st[i] = S.qs[0][i];
}

}  // namespace ygg
