// The fused step specialised for the common shape: readout rank 8, block 16, layer-input rank <= 16, table storage,
// one scale per tensor, at most 4 layers (every benchmark configuration). Same arithmetic and lane mapping as
// run_kernel (ygg_kernel.h); what changes is where the latency of one token goes:
//   - 4 streams per workgroup (one wavefront each) share LDS copies of what every stream reads at every token: the
//     unembedding Q of every layer, the layer-input down-projection V' of every routed layer, and the router rows of
//     the first descent round (the top 4 tree levels, nodes 1..15). That round then reads only LDS plus thresholds.
//   - the 15 thresholds of that first round, thr[x][1..15] for every routed layer, depend only on the token, so they
//     are loaded when the token is read, before the layer loop;
//   - the whole gather record of an expert (A16, U', P) and its table row are loaded in one burst as soon as the
//     expert is known (plain loads: non-temporal ones cut the fetched bytes by 6% but made the step 36% slower);
//   - LDS exchanges inside a stream's wavefront are ordered by wave-level fences instead of workgroup barriers, so the
//     4 streams of a workgroup never wait for each other.
#pragma once
#include "ygg_kernel.h"

namespace ygg {

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kFastWaves = 4;

template <int N, int L>
__global__ __launch_bounds__(64 * kFastWaves) __attribute__((amdgpu_waves_per_eu(4))) void fast_kernel(const YggDevModel m, const int32_t *__restrict__ tokens,
                                                               int B, int T, int8_t *__restrict__ state,
                                                               float *__restrict__ logits,
                                                               int32_t *__restrict__ leaves,
                                                               int8_t *__restrict__ states,
                                                               unsigned long long *__restrict__ digest) {
    constexpr int R = 8, BLK = 16, W = kFastWaves;
    constexpr int C = Lanes<N>::C, NL = Lanes<N>::NL;
    constexpr int Q4 = N / 4, QW = Q4 / 4;
    constexpr int QA = (Q4 % 16 == 0) ? 16 : 8;
    constexpr int RL = ReadoutLanes<N, R>::RL, SP = ReadoutLanes<N, R>::SP, GP = ReadoutLanes<N, R>::GP;
    constexpr int SPW = SP / 4;
    constexpr int AW = C * BLK / 2, NA = AW / 4;
    constexpr int LR = L > 1 ? L - 1 : 1;         // routed layers (array extent)
    constexpr float kInvN = 1.0f / (float)N;

    __shared__ __attribute__((aligned(16))) int8_t Qs[L][256 * R];
    __shared__ __attribute__((aligned(16))) int8_t Ws[LR][15 * N];
    __shared__ __attribute__((aligned(16))) int8_t Vs[LR][16 * N];
    __shared__ __attribute__((aligned(16))) int8_t qsw[W][L * N];
    __shared__ __attribute__((aligned(16))) int8_t zlw[W][16];
    __shared__ __attribute__((aligned(16))) int8_t zqw[W][16];

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int s = blockIdx.x * W + wv;
    const int V = m.V, VP = m.VP, E = m.E, D = m.D, R2 = m.R2;

    // the shared tables, once per workgroup
#pragma unroll
    for (int l = 0; l < L; l++) {
        const uint32_t *src = (const uint32_t *)m.layers[l].Q;
        uint32_t *dst = (uint32_t *)Qs[l];
        for (int i = tid; i < VP * R / 4; i += 64 * W) dst[i] = src[i];
    }
#pragma unroll
    for (int l = 1; l < L; l++) {
        const YggDevLayer &y = m.layers[l];
        const int rows = (1 << m.round_h[0]) - 1;     // the first round's block: slots 0 .. 2^h0 - 2
        const uint32_t *ws = (const uint32_t *)y.w;
        uint32_t *wd = (uint32_t *)Ws[l - 1];
        for (int i = tid; i < 15 * N / 4; i += 64 * W) wd[i] = i < rows * N / 4 ? ws[i] : 0u;
        uint32_t *vd = (uint32_t *)Vs[l - 1];
        if (R2 > 0) {
            const uint32_t *vs = (const uint32_t *)y.vl;
            for (int i = tid; i < 16 * N / 4; i += 64 * W) vd[i] = vs[i];
        } else {
            for (int i = tid; i < 16 * N / 4; i += 64 * W) vd[i] = 0u;
        }
    }
    __syncthreads();
    if (s >= B) return;

    int8_t *qs = qsw[wv];
    int8_t *zls = zlw[wv];
    int8_t *zqs = zqw[wv];
    const int qk = lane & 3, qj = lane >> 2;
    const int rj = lane / RL, rk = lane % RL;

    int8_t *st = state + (size_t)s * L * N;
    for (int i = lane; i < L * N; i += 64) qs[i] = st[i];
    if (lane < 16) zls[lane] = 0;
    wave_sync();
    unsigned long long dg = digest ? digest[s] : 0ull;
    const int32_t *tok = tokens + (size_t)s * T;
    int x_next = T > 0 ? tok[0] : 0;
    const int h1 = m.round_h[0], nn1 = (1 << h1) - 1;

    for (int t = 0; t < T; t++) {
        const int x = x_next;
        if (t + 1 < T) x_next = tok[t + 1];
        if (x < 0 || x >= V) {
            if (lane == 0) atomicOr(m.err, 1u);
            break;
        }
        // thresholds of the first router round of every routed layer
        float th1[LR];
#pragma unroll
        for (int l = 1; l < L; l++) th1[l - 1] = qj < nn1 ? m.layers[l].thr[(size_t)x * m.layers[l].thr_stride + qj] : 0.0f;
        float lg[4];
#pragma unroll
        for (int u = 0; u < 4; u++) lg[u] = 4 * lane + u < VP ? m.output_bias[4 * lane + u] : 0.0f;

#pragma unroll
        for (int l = 0; l < L; l++) {
            const YggDevLayer &y = m.layers[l];
            int r = x;
            float rho = 0.0f;
            uint32_t qbw[QW];
            if (l > 0) {
                const int8_t *qb = qs + (l - 1) * N;
                load_words<QW, QA>(qbw, qb + qk * Q4);
                int sg = 0;
                if (lane < N / 16) {
                    uint32_t g4[4];
                    load_words<4, 16>(g4, qb + 16 * lane);
#pragma unroll
                    for (int i = 0; i < 4; i++) sg = dot4(g4[i], g4[i], sg);
                }
                int S = 0;
#pragma unroll
                for (int g = 0; g < N / 16; g++) S += __builtin_amdgcn_readlane(sg, g);
                rho = 1.0f / sqrtf((float)S * kInvN + y.rms_eps);
                // first router round: nodes 1..15 from LDS, thresholds already loaded
                int ix = 1;
                {
                    int dot = 0;
                    if (qj < nn1) {
                        uint32_t wvv[QW];
                        load_words<QW, QA>(wvv, Ws[l - 1] + qj * N + qk * Q4);
#pragma unroll
                        for (int i = 0; i < QW; i++) dot = dot4(wvv[i], qbw[i], dot);
                    }
                    dot = sum4(dot);
                    const bool right = (float)dot * rho > th1[l - 1];
                    const unsigned long long mask = __ballot(right && qk == 0 && qj < nn1);
                    int loc = 0;
                    for (int lev = 0; lev < h1; lev++) loc = 2 * loc + 1 + (int)((mask >> (4 * loc)) & 1ull);
                    ix = (1 << h1) + (loc - nn1);
                }
                const float *thr = y.thr + (size_t)x * y.thr_stride;
                int base = 1 << h1, d0 = h1;
                for (int rd = 1; rd < m.n_rounds; rd++) {
                    const int h = m.round_h[rd];
                    const int nn = (1 << h) - 1;
                    const int slot = base + ((ix - (1 << d0)) << h) + qj;
                    int dot = 0;
                    float th = 0.0f;
                    if (qj < nn) {
                        uint32_t wvv[QW];
                        load_words<QW, QA>(wvv, y.w + (size_t)slot * N + qk * Q4);
                        th = thr[slot];
#pragma unroll
                        for (int i = 0; i < QW; i++) dot = dot4(wvv[i], qbw[i], dot);
                    }
                    dot = sum4(dot);
                    const bool right = (float)dot * rho > th;
                    const unsigned long long mask = __ballot(right && qk == 0 && qj < nn);
                    int loc = 0;
                    for (int lev = 0; lev < h; lev++) loc = 2 * loc + 1 + (int)((mask >> (4 * loc)) & 1ull);
                    base += (1 << d0) << h;
                    d0 += h;
                    ix = (ix << h) + (loc - nn);
                }
                r = ix - E;
            }

            // the expert's whole gather record and table row, in one burst
            const uint8_t *g = y.gath + (size_t)r * y.gath_bytes;
            uint32_t aw[AW], pw[SPW], uw[4][C];
            int trow[C];
            if (lane < NL) {
#pragma unroll
                for (int c = 0; c < NA; c++) {
                    const uint4 v = load16<false>(g + (c * NL + lane) * 16);
                    aw[4 * c] = v.x; aw[4 * c + 1] = v.y; aw[4 * c + 2] = v.z; aw[4 * c + 3] = v.w;
                }
                if (l > 0) {
#pragma unroll
                    for (int k4 = 0; k4 < 4; k4++) {
                        if (k4 < R2 / 4) {
                            uint32_t tmp[C];
                            load_words_sel<false, C, 4 * C>(tmp, g + y.off_U + ((size_t)(k4 * NL + lane) * C) * 4);
#pragma unroll
                            for (int c = 0; c < C; c++) uw[k4][c] = tmp[c];
                        }
                    }
                }
                const int16_t *tr = y.table + (size_t)r * y.table_sr + (size_t)x * y.table_sx + C * lane;
#pragma unroll
                for (int c = 0; c < C; c++) trow[c] = load_i16<false>(tr + c);
            }
            {
                const uint8_t *pp = g + y.off_P;
#pragma unroll
                for (int gi = 0; gi < SP / GP; gi++) {
                    uint32_t tmp[GP / 4];
                    load_words_sel<false, GP / 4, GP>(tmp, pp + (gi * 64 + lane) * GP);
#pragma unroll
                    for (int i = 0; i < GP / 4; i++) pw[gi * (GP / 4) + i] = tmp[i];
                }
            }

            // layer input zl from the LDS copy of V'
            if (l > 0 && R2 > 0) {
                uint32_t vv[QW];
                load_words<QW, QA>(vv, Vs[l - 1] + qj * N + qk * Q4);
                int a = 0;
#pragma unroll
                for (int i = 0; i < QW; i++) a = dot4(vv[i], qbw[i], a);
                a = sum4(a);
                if (qk == 0) {
                    float zf = (float)a * y.mv[qj];
                    zf = zf * rho;
                    zls[qj] = (int8_t)clamp127(cvt_rne(zf));
                }
            }
            wave_sync();

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
                    acc[c] = wadd((a + (1 << (m.shift - 1))) >> m.shift, trow[c]);
                }
                if (l > 0 && R2 > 0) {
                    int d[C];
#pragma unroll
                    for (int c = 0; c < C; c++) d[c] = 0;
#pragma unroll
                    for (int k4 = 0; k4 < 4; k4++) {
                        if (k4 < R2 / 4) {
                            const uint32_t zw = ((const uint32_t *)zls)[k4];
#pragma unroll
                            for (int c = 0; c < C; c++) d[c] = dot4(uw[k4][c], zw, d[c]);
                        }
                    }
#pragma unroll
                    for (int c = 0; c < C; c++) acc[c] = wadd(acc[c], cvt_rne((float)d[c] * y.layer_input_scale));
                }
#pragma unroll
                for (int c = 0; c < C; c++) qn[c] = sat8(acc[c]);
            }
            wave_sync();
            if (lane < NL) {
#pragma unroll
                for (int c = 0; c < C; c++) qs[l * N + C * lane + c] = (int8_t)qn[c];
            }
            wave_sync();

            {
                uint32_t qv[SPW];
                load_words<SPW, (SP % 16 == 0 ? 16 : (SP % 8 == 0 ? 8 : 4))>(qv, qs + l * N + rk * SP);
                int z = 0;
#pragma unroll
                for (int i = 0; i < SPW; i++) z = dot4(pw[i], qv[i], z);
                z = group_sum<RL>(z);
                if (rk == 0) zqs[rj] = (int8_t)clamp127(cvt_rne((float)z * y.readout_scale));
            }
            wave_sync();
            if (4 * lane < VP) {
                uint32_t zw[2];
                load_words<2, 16>(zw, zqs);
                uint32_t qq[8];
                load_words<8, 16>(qq, Qs[l] + 4 * lane * R);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    int d = dot4(qq[2 * u], zw[0], 0);
                    d = dot4(qq[2 * u + 1], zw[1], d);
                    lg[u] = lg[u] + (float)d * y.unembed_scale;
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
            wave_sync();
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
        if (states) {
            int8_t *so = states + ((size_t)s * T + t) * L * N;
            for (int i = lane; i < L * N; i += 64) so[i] = qs[i];
        }
    }
    wave_sync();
    for (int i = lane; i < L * N; i += 64) st[i] = qs[i];
    if (digest && lane == 0) digest[s] = dg;
}

}  // namespace ygg
