// The leaf-grouped step: streams that take the same expert at a (token, layer) are updated together, the expert's
// record read once for the group, and groups of at least `mfma_min` streams contract on int8 MFMA. For the benchmark
// shape (n 128, readout rank 8, layer-input rank 16, block 16, table storage, tensor scales).
//
// A call runs every (token, layer) of B streams as a phase of three launches on the caller's stream (so that the
// whole call can be captured in one hipGraph):
//   grp_route   one wavefront per stream: the layer's expert (the router descent of fast_kernel on the state below,
//               which the phase before wrote) and the layer input zl; the leaves output
//   grp_plan    one workgroup: a counting sort of the streams by expert in LDS (a histogram whose LDS atomics give
//               each stream its index in its group, a scan for the groups' offsets, a scatter), and the tile list
//               (tiles of at most 16 streams of one expert)
//   grp_update  one wavefront per tile: the update, the readout (zq kept per stream and layer) and the digest of each
//               stream of the tile; at the last layer the logits of its streams (every layer's unembedding term in
//               layer order, cpu/ygg.cpp:457)
// A tile of at least mfma_min streams runs the transition, the layer input and the readout as 16x16 int8 MFMA
// contractions over its streams (grp_tile_mfma); smaller tiles run fast_kernel's per-stream update once per stream,
// the record staying in L2 between them (grp_tile_gemv). Same integer and f32 arithmetic as fast_kernel.
//
// A stream whose token is outside [0, V) stops at that token (error bit 0), as in the other kernels.
#pragma once
#include "ygg_kernel_fast.h"

namespace ygg {

typedef int v4i32 __attribute__((ext_vector_type(4)));

constexpr int kGrpTile = 16;        // streams per tile (the MFMA's 16 rows)
constexpr int kGrpSlots = 8;        // zq bytes per stream and layer (readout rank 8)

// The workspace of a grouped call (device memory): B streams, L layers.
constexpr int kGrpMaxExperts = 16384;      // experts (and tokens) per layer the plan's LDS histogram holds
struct GroupWS {
    int32_t *leaf;                  // [B] expert of the phase, -1: the stream has stopped
    int32_t *pos;                   // [B] index in its expert's group
    int32_t *stop;                  // [B] first token not processed (T until a bad token)
    int32_t *sorted;                // [B] stream ids in expert order
    int4 *tiles;                    // [2 B + 1] (expert, first index into sorted, streams, 0)
    int32_t *ntiles;                // [1]
    int8_t *zl;                     // [B][16] layer input of the phase
    int8_t *zq;                     // [B][L][8] readouts of the current token
};

// bytes of a workspace for B streams, L layers (each piece 256-byte aligned)
inline size_t group_ws_bytes(int B, int L) {
    auto al = [](size_t b) { return (b + 255) / 256 * 256; };
    return al(4 * (size_t)B) * 4 + al(16 * (size_t)(2 * B + 1)) + al(4) + al(16 * (size_t)B) +
           al((size_t)B * L * kGrpSlots);
}
inline GroupWS group_ws_carve(void *base, int B, int L) {
    auto al = [](size_t b) { return (b + 255) / 256 * 256; };
    uint8_t *p = (uint8_t *)base;
    GroupWS w;
    w.leaf = (int32_t *)p; p += al(4 * (size_t)B);
    w.pos = (int32_t *)p; p += al(4 * (size_t)B);
    w.stop = (int32_t *)p; p += al(4 * (size_t)B);
    w.sorted = (int32_t *)p; p += al(4 * (size_t)B);
    w.tiles = (int4 *)p; p += al(16 * (size_t)(2 * B + 1));
    w.ntiles = (int32_t *)p; p += al(4);
    w.zl = (int8_t *)p; p += al(16 * (size_t)B);
    w.zq = (int8_t *)p;
    return w;
}

// ------------------------------------------------------------------------------------------------- init, route, plan

// a call's start: every stream running
__global__ __launch_bounds__(256) void grp_init(int B, int T, GroupWS ws) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < B) ws.stop[i] = T;
}

template <int N, int R, int R2>
__global__ __launch_bounds__(256) void grp_route(const YggDevModel m, const int32_t *__restrict__ tokens, int B, int T,
                                                 int t, int l, const int8_t *__restrict__ state,
                                                 int32_t *__restrict__ leaves, GroupWS ws) {
    using SH = Shape<N, R, R2>;
    using F = SH;
    constexpr int RC = N / 16, SC = kLdsRow<N> / 16, VR = 15 + R2;     // first-round rows, then V' rows
    __shared__ __attribute__((aligned(16))) int8_t W0[15 * kLdsRow<N>];
    __shared__ __attribute__((aligned(16))) int8_t V0[R2 * kLdsRow<N>];
    __shared__ float mv0[R2];
    __shared__ __attribute__((aligned(16))) int8_t zlw[4][SH::ZL];
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int s = blockIdx.x * 4 + wv;
    const YggDevLayer &y = m.layers[l];
    if (l > 0) {
        // the layer's first-round rows and V' into LDS (all loads first)
        const int rows = (1 << m.round_h[0]) - 1;
        constexpr int K = (VR * RC + 255) / 256;
        uint4 v[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int c = tid + 256 * k;
            v[k] = make_uint4(0u, 0u, 0u, 0u);
            if (c < rows * RC) v[k] = ((const uint4 *)y.w)[c];
            else if (c >= 15 * RC && c < VR * RC) v[k] = ((const uint4 *)y.vl)[c - 15 * RC];
        }
        const float mvv = tid < R2 ? y.mv[tid] : 0.0f;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int c = tid + 256 * k;
            if (c < 15 * RC) ((uint4 *)W0)[(c / RC) * SC + c % RC] = v[k];
            else if (c < VR * RC) ((uint4 *)V0)[((c - 15 * RC) / RC) * SC + (c - 15 * RC) % RC] = v[k];
        }
        if (tid < R2) mv0[tid] = mvv;
    }
    __syncthreads();
    if (s >= B) return;
    if (t >= ws.stop[s]) {
        if (lane == 0) ws.leaf[s] = -1;
        return;
    }
    const int x = __builtin_amdgcn_readfirstlane(tokens[(size_t)s * T + t]);
    if (x < 0 || x >= m.V) {
        // (only the token layer sees a new token: the stream stops here)
        if (lane == 0) {
            atomicOr(m.err, 1u);
            ws.stop[s] = t;
            ws.leaf[s] = -1;
        }
        return;
    }
    int r = x;
    if (l > 0) {
        const int qj = lane >> 2, nn1 = (1 << m.round_h[0]) - 1;
        uint32_t qbw[F::QW];
        const float rho = below_and_rho<N>(qbw, state + ((size_t)s * m.L + l - 1) * N, y.rms_eps, lane);
        const float th0 = qj < nn1 ? y.thr[(size_t)x * y.thr_stride + qj] : 0.0f;
        r = descend<N>(m, y, W0, th0, qbw, rho, x, lane);
        layer_input<SH>(zlw[wv], V0, mv0, qbw, rho, lane);
        wave_sync();
        if (lane < 4) ((uint32_t *)(ws.zl + (size_t)s * 16))[lane] = ((const uint32_t *)zlw[wv])[lane];
    }
    if (lane == 0) {
        ws.leaf[s] = r;
        if (leaves) leaves[((size_t)s * T + t) * m.L + l] = r;
    }
}

// One workgroup of 1024 threads, E <= kGrpMaxExperts experts: the streams' positions in their groups (LDS atomics
// on the histogram; the order of a group's streams is immaterial, every stream's arithmetic is its own), the groups'
// offsets (thread k takes the experts k + 1024 j, their stream and tile counts scanned over the workgroup; the order
// of the groups is immaterial too), the tile list, the streams in expert order.
__global__ __launch_bounds__(1024) void grp_plan(int B, int E, GroupWS ws) {
    __shared__ int hist[kGrpMaxExperts];
    __shared__ int wsum[16], wtil[16];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int e = tid; e < E; e += 1024) hist[e] = 0;
    __syncthreads();
    constexpr int PL = 8;       // streams per thread and pass, their loads issued together
    for (int s0 = tid; s0 < B; s0 += 1024 * PL) {
        int rr[PL];
#pragma unroll
        for (int k = 0; k < PL; k++) rr[k] = s0 + 1024 * k < B ? ws.leaf[s0 + 1024 * k] : -1;
#pragma unroll
        for (int k = 0; k < PL; k++)
            if (rr[k] >= 0) ws.pos[s0 + 1024 * k] = atomicAdd(&hist[rr[k]], 1);
    }
    __syncthreads();
    int ns = 0, nt = 0;
    for (int e = tid; e < E; e += 1024) {
        const int c = hist[e];
        ns += c;
        nt += (c + kGrpTile - 1) / kGrpTile;
    }
    // inclusive scans over the wavefront, then over the 16 wavefront totals
    int is = ns, it = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int us = __shfl_up(is, o), ut = __shfl_up(it, o);
        if (lane >= o) {
            is += us;
            it += ut;
        }
    }
    if (lane == 63) {
        wsum[wv] = is;
        wtil[wv] = it;
    }
    __syncthreads();
    int bs = 0, bt = 0, tt = 0;
#pragma unroll
    for (int w = 0; w < 16; w++) {
        if (w < wv) {
            bs += wsum[w];
            bt += wtil[w];
        }
        tt += wtil[w];
    }
    int off = bs + is - ns, toff = bt + it - nt;
    for (int e = tid; e < E; e += 1024) {
        const int c = hist[e];
        for (int k = 0; k < c; k += kGrpTile)
            ws.tiles[toff++] = make_int4(e, off + k, c - k < kGrpTile ? c - k : kGrpTile, 0);
        hist[e] = off;          // (the group's offset, for the scatter)
        off += c;
    }
    if (tid == 0) *ws.ntiles = tt;
    __syncthreads();
    for (int s0 = tid; s0 < B; s0 += 1024 * PL) {
        int rr[PL], pp[PL];
#pragma unroll
        for (int k = 0; k < PL; k++) {
            const bool in = s0 + 1024 * k < B;
            rr[k] = in ? ws.leaf[s0 + 1024 * k] : -1;
            pp[k] = in ? ws.pos[s0 + 1024 * k] : 0;
        }
#pragma unroll
        for (int k = 0; k < PL; k++)
            if (rr[k] >= 0) ws.sorted[hist[rr[k]] + pp[k]] = s0 + 1024 * k;
    }
}

// ------------------------------------------------------------------------------------------------- update

// the per-stream outputs shared by both tile paths: the digest term of stream s (its new state at qn, LDS) and the
// logits of token t at the last layer (the earlier layers' zq of the token from ws.zq, this layer's from zqc in LDS,
// each through its unembedding, in layer order from the output bias). Lanes: the digest's coordinate sum over the
// wavefront; logits 4 classes per lane.
template <class SH>
__device__ __forceinline__ void grp_stream_out(const YggDevModel &m, const GroupWS &ws, int s, int r, int l, int t,
                                               int T, const int8_t *qn, const int8_t *zqc,
                                               unsigned long long *digest, float *logits, int lane) {
    constexpr int N = SH::N, L8 = kGrpSlots;
    if (digest) {
        uint32_t a = 0;
        for (int i = lane; i < N; i += 64) a += ((uint8_t)qn[i] + 1u) * (uint32_t)(2 * i + 1);
        a = wave_sum_u32(a);
        if (lane == 0)
            digest[s] = digest[s] * kDigestMul + ((unsigned long long)(uint32_t)r * kDigestLeaf +
                                                  (unsigned long long)a * kDigestCoord + (unsigned long long)l);
    }
    if (logits && l == m.L - 1) {
        const int VP = m.VP;
        float lg[4];
#pragma unroll
        for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? m.output_bias[4 * lane + u] : 0.0f;
        for (int j = 0; j < m.L; j++) {
            const YggDevLayer &yj = m.layers[j];
            const int8_t *zq = j == l ? zqc : ws.zq + ((size_t)s * m.L + j) * L8;
            uint32_t zw[2];
            zw[0] = ((const uint32_t *)zq)[0];
            zw[1] = ((const uint32_t *)zq)[1];
            if (4 * lane < VP) {
                // Q of classes 4 lane .. 4 lane + 3, class-major [VP][R] (8 bytes a class)
                const uint4 q0 = ((const uint4 *)yj.Q)[2 * lane], q1 = ((const uint4 *)yj.Q)[2 * lane + 1];
                const uint32_t qq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int d = dot4(qq[2 * u + 1], zw[1], dot4(qq[2 * u], zw[0], 0));
                    lg[u] = lg[u] + (float)d * yj.unembed_scale;
                }
            }
        }
        store_logits(logits + ((size_t)s * T + t) * m.V, lg, m.V, lane);
    }
}

// A tile on fast_kernel's per-stream code: for each stream, its table row and the expert's record (one record for
// the tile: only the table row differs between its streams), the update, the readout.
template <class SH>
__device__ __forceinline__ void grp_tile_gemv(const YggDevModel &m, const int32_t *tokens, int T, int t, int l,
                                              int8_t *state, int8_t *states, float *logits,
                                              unsigned long long *digest, const GroupWS &ws, int r, int first, int n,
                                              int8_t *qn, int8_t *zqs, int lane) {
    using F = SH;
    constexpr int N = SH::N;
    const YggDevLayer &y = m.layers[l];
    for (int i = 0; i < n; i++) {
        const int s = __builtin_amdgcn_readfirstlane(ws.sorted[first + i]);
        const int x = __builtin_amdgcn_readfirstlane(tokens[(size_t)s * T + t]);
        int8_t *q = state + ((size_t)s * m.L + l) * N;
        Gather<SH> G;
        gather<SH>(G, y, r, x, l > 0, lane);
        int qv[F::C];
        if (lane < F::NL) update<SH>(qv, G, q, ws.zl + (size_t)s * 16, y, l > 0, m.shift, lane);
        wave_sync();
        if (lane < F::NL) {
#pragma unroll
            for (int c = 0; c < F::C; c++) qn[F::C * lane + c] = (int8_t)qv[c];
        }
        wave_sync();
        readout<SH>(zqs, G.pw, qn, y.readout_scale, lane);
        wave_sync();
        if (lane < kGrpSlots && l < m.L - 1) ws.zq[((size_t)s * m.L + l) * kGrpSlots + lane] = zqs[lane];
        for (int k = lane; k < N; k += 64) q[k] = qn[k];
        if (states)
            for (int k = lane; k < N; k += 64) states[(((size_t)s * T + t) * m.L + l) * N + k] = qn[k];
        grp_stream_out<SH>(m, ws, s, r, l, t, T, qn, zqs, digest, logits, lane);
        wave_sync();
    }
}

// ------------------------------------------------------------------------------------------------- MFMA tile
// One wavefront, up to 16 streams of one expert as the 16 rows of v_mfma_i32_16x16x32_i8 / 16x16x64_i8 (row m of
// the A operand and column n of the B operand in lane m (n) mod 16, the reduction index split over the lane's bytes
// and lane / 16 the same way in both operands; the 4 results of lane l are rows 4 (l / 16) + e, column l mod 16).
// The expert's record is staged in LDS once for the tile, with the tile's old states and table rows.
//   transition, block b (coordinates 16 b .. 16 b + 15): D = Q_b hi^T, then D = Q_b lo^T + (D << 8): A16 q exactly,
//     as the per-stream code's two dot chains (reduction over the block's 16 columns, the upper half of K zero)
//   layer input: D = ZL U'_b^T (reduction over the 16 ranks)
//   readout: Z = Q_new P^T on the 16x16x64 form (reduction over the 128 coordinates, columns 8..15 zero)
//   logits (last layer): per 16 classes and layer, ZQ_j Q_j^T (reduction over the 8 ranks), added to the output
//     bias in layer order as f32, as the per-stream code does
// Rows past the tile's streams repeat its last stream (their loads stay in bounds) and write nothing.
constexpr int kGrpRec = 7168;       // gather record bytes of the shape (A 4096, P 1024, U' 2048)
constexpr int kQsRow = 144, kTbRow = 272;       // LDS row strides of states and table rows (16-byte multiples)
struct MfmaLds {
    int8_t rec[kGrpRec];
    int8_t qs[kGrpTile * kQsRow];
    int8_t tb[kGrpTile * kTbRow];
    int8_t zq[kGrpTile * kGrpSlots];
};

__device__ __forceinline__ v4i32 mfma_16x16x32(long a, long b, v4i32 c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4i32 mfma_16x16x64(v4i32 a, v4i32 b, v4i32 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <class SH>
__device__ __forceinline__ void grp_tile_mfma(const YggDevModel &m, const int32_t *tokens, int T, int t, int l,
                                              int8_t *state, int8_t *states, float *logits,
                                              unsigned long long *digest, const GroupWS &ws, int r, int first, int n,
                                              MfmaLds &S, int lane) {
    static_assert(SH::N == 128 && SH::R == 8 && SH::R2 == 16 && SH::BLK == 16, "the grouped step's shape");
    constexpr int N = SH::N;
    const YggDevLayer &y = m.layers[l];
    const bool routed = l > 0;
    const int L = m.L;
    const int rs = lane & 15, g = lane >> 4;       // operand row / column, reduction group
    const int si = lane >> 2, sp = lane & 3;       // staging: stream si, quarter sp of its row
    // the tile's streams: lane k < 16 holds stream k's id and token
    const int sid_r = ws.sorted[first + (rs < n ? rs : n - 1)];
    const int x_r = tokens[(size_t)sid_r * T + t];
    const int sid_s = __shfl(sid_r, si), x_s = __shfl(x_r, si);
    // every load first: the record, the states, the table rows, the layer inputs
    const uint8_t *gr = y.gath + (uint32_t)r * (uint32_t)y.gath_bytes;
    const int nch = (int)(y.gath_bytes >> 4);
    uint4 rv[kGrpRec / 16 / 64];
#pragma unroll
    for (int k = 0; k < kGrpRec / 16 / 64; k++) {
        const int c = lane + 64 * k;
        rv[k] = ((const uint4 *)gr)[c < nch ? c : nch - 1];
    }
    const uint4 *qsrc = (const uint4 *)(state + ((size_t)sid_s * L + l) * N + 32 * sp);
    const uint4 q0 = qsrc[0], q1 = qsrc[1];
    const uint4 *tsrc = (const uint4 *)(y.table + ((uint32_t)r * (uint32_t)y.table_sr +
                                                   (uint32_t)x_s * (uint32_t)y.table_sx) + 32 * sp);
    uint4 tv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) tv[k] = tsrc[k];
    long za = 0;
    if (routed) {
        const long zv = *(const long *)(ws.zl + (size_t)sid_r * 16 + 8 * (g & 1));
        za = g < 2 ? zv : 0;
    }
#pragma unroll
    for (int k = 0; k < kGrpRec / 16 / 64; k++) {
        const int c = lane + 64 * k;
        if (c < nch) ((uint4 *)S.rec)[c] = rv[k];
    }
    ((uint4 *)(S.qs + si * kQsRow + 32 * sp))[0] = q0;
    ((uint4 *)(S.qs + si * kQsRow + 32 * sp))[1] = q1;
#pragma unroll
    for (int k = 0; k < 4; k++) ((uint4 *)(S.tb + si * kTbRow + 64 * sp))[k] = tv[k];
    wave_sync();

    // the update, block by block, in place in S.qs (block b's A operand is read before its results are written)
    const v4i32 zero = {0, 0, 0, 0};
    const int half = 1 << (m.shift - 1);
#pragma unroll
    for (int b = 0; b < N / 16; b++) {
        const int i = 16 * b + rs;                  // this lane's column: coordinate i
        const long qa = g < 2 ? *(const long *)(S.qs + rs * kQsRow + 16 * b + 8 * g) : 0;
        const int8_t *hi = S.rec + ((2 * (i & 1)) * 64 + (i >> 1)) * 16 + 8 * (g & 1);
        const long bh = g < 2 ? *(const long *)hi : 0, bl = g < 2 ? *(const long *)(hi + 1024) : 0;
        v4i32 d = mfma_16x16x32(qa, bh, zero);
        d = d << 8;
        d = mfma_16x16x32(qa, bl, d);
        v4i32 du = zero;
        if (routed) {
            const int8_t *uw = S.rec + y.off_U + ((2 * (g & 1)) * 128 + i) * 4;
            const long bu = g < 2 ? (long)(((unsigned long)*(const uint32_t *)(uw + 512) << 32) |
                                           *(const uint32_t *)uw) : 0;
            du = mfma_16x16x32(za, bu, zero);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int s = 4 * g + e;
            const int in = *(const int16_t *)(S.tb + s * kTbRow + 2 * i);
            int acc = wadd((d[e] + half) >> m.shift, in);
            if (routed) acc = wadd(acc, cvt_rne((float)du[e] * y.layer_input_scale));
            S.qs[s * kQsRow + i] = (int8_t)sat8(acc);
        }
    }
    wave_sync();
    // the readout: zq[s][j] = clamp(rint(f32(P_j q_new) m_z), +-127)
    {
        v4i32 z = zero;
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
            const v4i32 qa = *(const v4i32 *)(S.qs + rs * kQsRow + 64 * kc + 16 * g);
            const v4i32 pv = *(const v4i32 *)(S.rec + y.off_P + (rs & 7) * 128 + 64 * kc + 16 * g);
            z = mfma_16x16x64(qa, rs < 8 ? pv : zero, z);
        }
        if (rs < kGrpSlots) {
#pragma unroll
            for (int e = 0; e < 4; e++)
                S.zq[(4 * g + e) * kGrpSlots + rs] = (int8_t)clamp127(cvt_rne((float)z[e] * y.readout_scale));
        }
    }
    wave_sync();
    // per-stream outputs: the new state (and states), the zq of this layer, the digest term
    if (si < n) {
        const uint4 n0 = ((const uint4 *)(S.qs + si * kQsRow + 32 * sp))[0];
        const uint4 n1 = ((const uint4 *)(S.qs + si * kQsRow + 32 * sp))[1];
        uint4 *qd = (uint4 *)(state + ((size_t)sid_s * L + l) * N + 32 * sp);
        qd[0] = n0;
        qd[1] = n1;
        if (states) {
            uint4 *sd = (uint4 *)(states + (((size_t)sid_s * T + t) * L + l) * N + 32 * sp);
            sd[0] = n0;
            sd[1] = n1;
        }
    }
    if (lane < n && l < L - 1)
        *(uint2 *)(ws.zq + ((size_t)sid_r * L + l) * kGrpSlots) = *(const uint2 *)(S.zq + lane * kGrpSlots);
    if (digest) {
        uint32_t a = 0;
#pragma unroll 8
        for (int k = 0; k < 32; k++) {
            const int c = 32 * sp + k;
            a += ((uint8_t)S.qs[si * kQsRow + c] + 1u) * (uint32_t)(2 * c + 1);
        }
        a = (uint32_t)sum4((int)a);
        if (sp == 0 && si < n)
            digest[sid_s] = digest[sid_s] * kDigestMul + ((unsigned long long)(uint32_t)r * kDigestLeaf +
                                                          (unsigned long long)a * kDigestCoord +
                                                          (unsigned long long)l);
    }
    // the logits at the last layer: per 16 classes, every layer's Q_j zq_j in layer order from the output bias
    if (logits && l == L - 1) {
        long zj[YGG_MAX_LAYERS];
        for (int j = 0; j < L; j++) {
            const int8_t *src = j == l ? S.zq + rs * kGrpSlots : ws.zq + ((size_t)sid_r * L + j) * kGrpSlots;
            const long v = *(const long *)src;
            zj[j] = g == 0 ? v : 0;
        }
        int sidd[4];
#pragma unroll
        for (int e = 0; e < 4; e++) sidd[e] = __shfl(sid_r, 4 * g + e);
        const int V = m.V;
        for (int cb = 0; cb < m.VP / 16; cb++) {
            const int c = 16 * cb + rs;
            const float bias = m.output_bias[c];
            float lg[4] = {bias, bias, bias, bias};
            for (int j = 0; j < L; j++) {
                const YggDevLayer &yj = m.layers[j];
                const long qv = *(const long *)(yj.Q + (size_t)c * kGrpSlots);
                const v4i32 d = mfma_16x16x32(zj[j], g == 0 ? qv : 0, zero);
#pragma unroll
                for (int e = 0; e < 4; e++) lg[e] = lg[e] + (float)d[e] * yj.unembed_scale;
            }
            if (c < V) {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (4 * g + e < n) logits[((size_t)sidd[e] * T + t) * V + c] = lg[e];
            }
        }
    }
}

template <int N, int R, int R2>
__global__ __launch_bounds__(256) void grp_update(const YggDevModel m, const int32_t *__restrict__ tokens, int B,
                                                  int T, int t, int l, int8_t *__restrict__ state,
                                                  int8_t *__restrict__ states, float *__restrict__ logits,
                                                  unsigned long long *__restrict__ digest, GroupWS ws, int mfma_min) {
    using SH = Shape<N, R, R2>;
    __shared__ __attribute__((aligned(16))) MfmaLds ml[4];
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int waves = gridDim.x * 4;
    const int ntiles = __builtin_amdgcn_readfirstlane(*ws.ntiles);
    for (int k = blockIdx.x * 4 + wv; k < ntiles; k += waves) {
        const int4 tl = ws.tiles[k];
        const int r = __builtin_amdgcn_readfirstlane(tl.x), first = __builtin_amdgcn_readfirstlane(tl.y);
        const int n = __builtin_amdgcn_readfirstlane(tl.z);
        if (mfma_min > 0 && n >= mfma_min)
            grp_tile_mfma<SH>(m, tokens, T, t, l, state, states, logits, digest, ws, r, first, n, ml[wv], lane);
        else
            grp_tile_gemv<SH>(m, tokens, T, t, l, state, states, logits, digest, ws, r, first, n, ml[wv].qs,
                              ml[wv].zq, lane);
        wave_sync();
    }
}

}  // namespace ygg
