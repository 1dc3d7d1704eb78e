// Speculative generation for one stream (kModeGenSpec; included by ygg_kernel_fast.h before fast_body, whose
// per-layer pieces it uses).
//
// Generation is a chain: the token sampled after step t is the input of step t + 1, so every layer of step t + 1
// waits for all layers of step t. Only two things tie step t + 1 to step t, though: the sampled token x(t + 1), which
// is one of V values, and the states of the layers. So while the stream finishes step t, helper wavefronts compute
// step t + 1's first layers for every candidate token at once: given the states of layers 0 .. S - 1 after step t,
// the helper of candidate x updates the token layer with expert x, descends the router of layer 1 with x's
// thresholds, updates layer 1, ... up to layer S's router descent and layer input, and leaves the new states, the
// readouts zq, layer S's leaf and its layer input in x's slot. The stream then samples x(t + 1), reads x's slot and
// starts step t + 1 at layer S's update: the token layer and S router descents leave its chain.
//
// Exchange. Every exchanged word travels in an 8-byte unit with a 32-bit tag, the epoch of the step it belongs to
// (the call's first epoch, from a host counter, plus the step index), stored with one 64-bit store (single-copy
// atomic). A reader takes a block only when every unit carries the epoch it expects, so a unit that is stale, torn
// by a concurrent writer or left by another call is never used; the stream computes the step itself instead, with
// the same code as without helpers, and every result is the same bit for bit either way.
//   - token unit: the stream stores its input x(t) of step t as soon as it has sampled it (tag E0 + t);
//   - slot of x: the helper of x stores step t + 1's results for x (tag E0 + t + 1), the states of layers
//     0 .. S - 1 in every copy. A step the stream computes itself (the first, or one whose slot did not come in
//     time) it stores the same states into the slot of its input (tag E0 + t), as a helper would have.
// The helpers of step t + 1 thus read the states after step t from the slot of x(t) as soon as its helper has stored
// them, not after the stream has taken them: the stream's own poll is off their chain.
// Stores and loads are at device scope (written through past the XCD's L2, read past it), coherent between XCDs:
// each XCD has its own L2, and 255 helpers on the stream's XCD alone move about 9 MB per step through that XCD's
// share of the fabric, which measured twice as slow a chain for every helper and for the stream itself (10.4 us a
// step); spread over the 8 XCDs they move about 1 MB each.
//
// Waiting. The stream never waits on a helper beyond a short bounded poll of its slot (then it computes). Every
// helper wait is bounded by the wall clock and a helper that times out leaves, so every wavefront ends; a helper that
// finds the slot it waits for already rewritten for a later step skips to the next token.
//
// Placement. Workgroup 0 runs the stream, workgroups 1 .. H help (the dispatcher hands workgroups to the XCDs in
// turn: workgroup i runs on XCD i mod 8, each on a CU of its own, as read from the hardware XCC and CU ids). All 4
// wavefronts of a helper workgroup stage the LDS tables; then one of them helps, or two in the first spec_pairs(H, V)
// workgroups, so that H workgroups cover up to 2 H candidates, and the others leave (one helper wavefront per CU made
// the descents faster: configuration 4's 1.9 us with four, 1.3 with two, 1.16 with one). The stream workgroup's 3
// staging wavefronts help too, one candidate each (those past the last candidate leave); with more candidates than
// helpers the uncovered ones change with every step (candidate (j + step) mod V for helper j of nh). Every workgroup
// holds the build's LDS: with the deep descent's second-round rows (the stream's and the helpers' descents both read
// them from LDS), one workgroup per CU.
#pragma once

namespace ygg {

// of h helper workgroups for V candidates, the first spec_pairs(h, V) run two helper wavefronts, the others one (one
// candidate per wavefront, as many as fit)
__host__ __device__ constexpr int spec_pairs(int h, int V) { return V <= h ? 0 : (V - h > h ? h : V - h); }
// helper wavefronts of h helper workgroups: theirs and the stream workgroup's staging wavefronts
__host__ __device__ constexpr int spec_helper_waves(int h, int V) { return h + spec_pairs(h, V) + kFastWaves - 1; }
// the helper index of wavefront wv of helper workgroup b (1 .. h), or -1 for a wavefront that does not help
__device__ __forceinline__ int spec_helper_index(int b, int wv, int h, int V) {
    const int p = spec_pairs(h, V);
    if (b <= p) return wv < 2 ? 2 * (b - 1) + wv : -1;
    return wv < 1 ? p + b - 1 : -1;
}

// routed layers whose descent the helpers take over: 1 for a 2-layer model, 2 for 3 or 4 layers, 3 for 5 (the
// stream then keeps two layers, as with 4: with 2 the stream's side of 5 layers set the period, 6.8 us/token on the
// reference's small shape, 7.1 on its medium one and 12.8 on its large one against 4.9, 5.3 and 10.6 with 3)
template <int L> constexpr int kSpecDepth = L > 4 ? 3 : (L > 2 ? 2 : 1);

template <class SH, int S> struct SpecLayout {
    static constexpr int PW = S * SH::N / 4;                                   // state words (in every copy)
    static constexpr int KP = (PW + 63) / 64;                                  // their units per lane
    static constexpr int SW = S * SH::N / 4 + S * SH::R / 4 + 1 + SH::R2P / 4;  // slot words
    static constexpr int KS = (SW + 63) / 64;
    static constexpr int TB = S * SH::R + 4 + SH::ZL;    // LDS bytes of a slot after the states: zq .., leaf, zl
    static_assert(KP <= 4 && KS <= 4 && KS * 64 <= kSpecCopyUnits, "units per lane");
};

__device__ __forceinline__ uint64_t spec_unit(uint32_t tag, uint32_t word) { return (uint64_t)word << 32 | tag; }
__device__ __forceinline__ uint64_t spec_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void spec_store(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void spec_count(uint64_t *area, int which, unsigned long long v) {
    atomicAdd((unsigned long long *)(area + kSpecStats + which), v);
}

// wall-clock bound (100 MHz ticks)
constexpr uint64_t kSpecPubWait = 20000;       // 200 us between two steps' states

// The helper wavefront j of nh: serves every step of this call from the first (relative epoch 0) to T - 2: for the
// stream's input xe of step e (its token unit), it reads the states after step e from xe's slot (copy `copy`) and
// computes step e + 1 for its candidate. qh: this wavefront's LDS states, new states of layers 0 .. S - 1 at qh (the
// slot's order), the old ones at qh + S N; sp: the slot's tail (zq of layers 0 .. S - 1, layer S's leaf, its layer
// input). DEEP: the routed layers' second-round rows are in LDS from W1 on (load_round2's layout: kR2Slots N bytes a
// layer, fast_kernel's deep descent), else read from global memory. Every helper wavefront polls on its own.
template <class SH, int L, bool GROUP, bool DEEP>
__device__ __forceinline__ void spec_helper(const YggDevModel &m, const YggIO &io, int T, int j, int nh,
                                            const SharedTables<SH, L> &St, const GroupTablesOf<SH, L, GROUP> &GT,
                                            const int8_t *W1, int8_t *qh, int8_t *sp, int lane, int copy) {
    constexpr int N = SH::N, R = SH::R, S = kSpecDepth<L>;
    using LY = SpecLayout<SH, S>;
    using F = SH;
    uint64_t *const area = io.spec;
    const uint32_t E0 = io.spec_epoch;
    // (no step to serve, or no candidate: past the vocabulary while every candidate has a wavefront)
    if (T < 2 || j >= nh || (nh >= m.V && j >= m.V)) return;
    const uint32_t span = (uint32_t)T - 2;        // relative epochs worth serving
    const uint64_t *tokp = area + kSpecTok + (size_t)copy * kSpecCopyUnits;
    if (lane == 0) spec_count(area, 3, 1);
    const int V = m.V;
    const int n2 = m.n_rounds > 1 ? 1 << (m.round_h[0] + m.round_h[1]) : 0;
    const int qj = lane >> 2, nn1 = (1 << m.round_h[0]) - 1;
    const Tail tl = make_tail(m, lane, (!DEEP && tail_fold(m)) ? 1 : 2);
    int8_t *const qnew = qh, *const qold = qh + S * N;
    int8_t *const zl = sp + S * R + 4;
    uint32_t next = 0;
    int served = 0;
    bool timed_out = false;
    // every candidate has a wavefront of its own (x = j at every epoch): its token-layer record and thresholds load
    // while the states are awaited
    const bool fixed = nh >= m.V;
    while (next <= span) {
        Gather<SH, false> G;
        float th1[S];
        float4 th2[S];
        // the token layer with expert x's record, then x's thresholds of the first two rounds of layers 1 .. S
        auto prefetch = [&](int xx) {
            gather<SH, GROUP, true, false>(G, m.layers[0], xx, xx, false, lane);
#pragma unroll
            for (int l = 1; l <= S; l++) {
                const YggDevLayer &y = m.layers[l];
                th1[l - 1] = qj < nn1 ? y.thr[(size_t)xx * y.thr_stride + qj] : 0.0f;
                th2[l - 1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (4 * lane < n2)
                    th2[l - 1] = *(const float4 *)(y.thr + (size_t)xx * y.thr_stride + (1 << m.round_h[0]) + 4 * lane);
            }
        };
        if (fixed) prefetch(j);
        // the newest token not served yet (epoch e, the stream's input xe of step e), then copy `copy` of xe's states
        // after step e in xe's slot: two looks in flight each (as in spec_take); the slot is whole when every unit
        // carries tag E0 + e, and a unit with a later tag means that the slot has been rewritten for a later step (this
        // wavefront is behind: it goes on to the next token)
        const uint64_t t0 = wall_clock64();
        uint32_t e = 0;
        int xe = 0;
        bool got = false;
        {
            auto fresh = [&](uint64_t d) {
                const uint32_t e0 = (uint32_t)d - E0;
                return e0 >= next && e0 <= span;
            };
            uint64_t a = spec_load(tokp), b;
            for (;;) {
                __builtin_amdgcn_s_sleep(1);
                b = spec_load(tokp);
                a = uniform_u64(a);
                if (fresh(a)) {
                    got = true;
                    break;
                }
                if (wall_clock64() - t0 > kSpecPubWait) break;
                __builtin_amdgcn_s_sleep(1);
                a = spec_load(tokp);
                b = uniform_u64(b);
                if (fresh(b)) {
                    a = b;
                    got = true;
                    break;
                }
                if (wall_clock64() - t0 > kSpecPubWait) break;
            }
            e = (uint32_t)a - E0;
            xe = (int)(uint32_t)(a >> 32);
        }
        if (!got) {
            timed_out = true;
            break;
        }
        // (the stream writes only tokens it sampled; the bound keeps every address in the area whatever a unit holds)
        if ((uint32_t)xe >= (uint32_t)V) xe = 0;
        uint64_t u[LY::KP];
        {
            const uint32_t tag = E0 + e;
            const uint64_t *src = area + kSpecSlots + (size_t)xe * kSpecSlotUnits + (size_t)copy * kSpecCopyUnits;
            uint64_t v[LY::KP];
            auto look = [&](uint64_t (&d)[LY::KP]) {
#pragma unroll
                for (int k = 0; k < LY::KP; k++) {
                    const int w = 64 * k + lane;
                    d[k] = w < LY::PW ? spec_load(src + w) : spec_unit(tag, 0u);
                }
            };
            // 1: whole, -1: rewritten for a later step, 0: not yet
            auto state = [&](const uint64_t (&d)[LY::KP]) {
                bool bad = false, late = false;
#pragma unroll
                for (int k = 0; k < LY::KP; k++) {
                    const int32_t dt = (int32_t)((uint32_t)d[k] - tag);
                    bad = bad || dt != 0;
                    late = late || dt > 0;
                }
                return lane_mask(late) != 0ull ? -1 : (lane_mask(bad) == 0ull ? 1 : 0);
            };
            int st = 0;
            look(u);
            for (;;) {
                __builtin_amdgcn_s_sleep(1);
                look(v);
                st = state(u);
                if (st != 0) break;
                if (wall_clock64() - t0 > kSpecPubWait) break;
                __builtin_amdgcn_s_sleep(1);
                look(u);
                st = state(v);
                if (st != 0) {
#pragma unroll
                    for (int k = 0; k < LY::KP; k++) u[k] = v[k];
                    break;
                }
                if (wall_clock64() - t0 > kSpecPubWait) break;
            }
            if (st == 0) {
                timed_out = true;
                break;
            }
            if (st < 0) {
                next = e + 1;
                continue;
            }
        }
        next = e + 1;
        const int x = nh >= V ? j : (int)((uint32_t)(j + e) % (uint32_t)V);
        if (x >= V) continue;
#pragma unroll
        for (int k = 0; k < LY::KP; k++) {
            const int w = 64 * k + lane;
            if (w < LY::PW) ((uint32_t *)qold)[w] = (uint32_t)(u[k] >> 32);
        }
        wave_sync();
        // the token layer with expert x (loaded above for a fixed candidate; else now, the thresholds after the
        // record, which the update's wait then leaves in flight)
        int qn[F::C];
        uint32_t ppw[F::SPW];      // the P granules and readout scale of the layer whose readout is pending
        float pmz;
        if (!fixed) prefetch(x);
        {
            const YggDevLayer &y = m.layers[0];
            const float *mul = nullptr;
            if constexpr (GROUP) mul = GT.mul[0];
            if (lane < F::NL) update<SH, GROUP, false, false>(qn, G, qold, zl, y, false, m.shift, lane, mul);
            wave_sync();
            if (lane < F::NL) {
#pragma unroll
                for (int c = 0; c < F::C; c++) qnew[F::C * lane + c] = (int8_t)qn[c];
            }
            wave_sync();
#pragma unroll
            for (int i = 0; i < F::SPW; i++) ppw[i] = G.pw[i];
            pmz = GROUP ? G.mzr : y.readout_scale;
        }
        // layers 1 .. S - 1 whole, layer S's descent and layer input; the readout of layer l - 1 runs while layer
        // l's last router round is loading
#pragma unroll
        for (int l = 1; l <= S; l++) {
            const YggDevLayer &y = m.layers[l];
            uint32_t qbw[F::QW];
            float rho = below_and_rho<N>(qbw, qnew + (l - 1) * N, y.rms_eps, lane);
            if constexpr (GROUP)
                if (y.r2b) rho = group_rho<N>(qbw, GT.r2[l - 1], y.rms_eps);
            auto hook = [&]() { readout<SH>(sp + (l - 1) * R, ppw, qnew + (l - 1) * N, pmz, lane); };
            int r;
            if constexpr (DEEP)
                r = descend_deep<N, decltype(hook)>(m, y, St.W[l - 1], th1[l - 1], W1 + (l - 1) * kR2Slots<N> * N,
                                                    th2[l - 1], qbw, qnew + (l - 1) * N, rho, x, lane, tl, hook);
            else
                r = descend_deep<N, decltype(hook), true>(m, y, St.W[l - 1], th1[l - 1],
                                                          y.w + ((size_t)1 << m.round_h[0]) * N, th2[l - 1], qbw,
                                                          qnew + (l - 1) * N, rho, x, lane, tl, hook);
            if (l < S) gather<SH, GROUP, true, false>(G, y, r, x, true, lane);
            layer_input<SH>(zl, St.V[l - 1], St.mv[l - 1], qbw, rho, lane);
            wave_sync();
            if (l == S) {
                if (lane == 0) *(int32_t *)(sp + S * R) = r;
                break;
            }
            const float *mul = nullptr;
            if constexpr (GROUP) mul = GT.mul[l - 1];
            if (lane < F::NL) update<SH, GROUP, false, false>(qn, G, qold + l * N, zl, y, true, m.shift, lane, mul);
            wave_sync();
            if (lane < F::NL) {
#pragma unroll
                for (int c = 0; c < F::C; c++) qnew[l * N + F::C * lane + c] = (int8_t)qn[c];
            }
            wave_sync();
#pragma unroll
            for (int i = 0; i < F::SPW; i++) ppw[i] = G.pw[i];
            pmz = GROUP ? G.mzr : y.readout_scale;
        }
        wave_sync();
        // x's slot: step e + 1's results
        uint64_t *slot = area + kSpecSlots + (size_t)x * kSpecSlotUnits;
#pragma unroll
        for (int k = 0; k < LY::KS; k++) {
            const int w = 64 * k + lane;
            if (w < LY::SW) {
                const uint32_t word = w < S * N / 4 ? ((const uint32_t *)qnew)[w]
                                                    : ((const uint32_t *)sp)[w - S * N / 4];
                const uint64_t v = spec_unit(E0 + e + 1, word);
                spec_store(slot + w, v);
                if (w < LY::PW) {
#pragma unroll
                    for (int c = 1; c < kSpecCopies; c++) spec_store(slot + c * kSpecCopyUnits + w, v);
                }
            }
        }
        served++;
    }
    if (lane == 0) {
        if (served) spec_count(area, 2, 1);
        if (timed_out) spec_count(area, 4, 1);
    }
}

// The stream's side. spec_take: x's slot for step t (tag E0 + t), polled for at most `wait` ticks; when every unit
// carries the tag, the states of layers 0 .. S - 1 go to qs (the stream's state rows), the rest to sp, layer S's
// leaf to `leaf`, and it returns true.
template <class SH, int S>
__device__ __forceinline__ bool spec_take(const YggIO &io, int x, int t, int8_t *qs, int8_t *sp, int lane,
                                          uint64_t wait, int &leaf) {
    using LY = SpecLayout<SH, S>;
    constexpr int N = SH::N, LW = S * SH::N / 4 + S * SH::R / 4;     // the leaf's word
    const uint32_t tag = io.spec_epoch + (uint32_t)t;
    const uint64_t *slot = io.spec + kSpecSlots + (size_t)x * kSpecSlotUnits;
    // two looks in flight: the next is issued before the last one is examined, so that the slot is seen about one
    // load latency after it lands (a look-wait-look loop sees it up to two later)
    uint64_t u[LY::KS], v[LY::KS];
    auto look = [&](uint64_t (&d)[LY::KS]) {
#pragma unroll
        for (int k = 0; k < LY::KS; k++) {
            const int w = 64 * k + lane;
            d[k] = w < LY::SW ? spec_load(slot + w) : spec_unit(tag, 0u);
        }
    };
    auto whole = [&](const uint64_t (&d)[LY::KS]) {
        bool bad = false;
#pragma unroll
        for (int k = 0; k < LY::KS; k++) bad = bad || (uint32_t)d[k] != tag;
        return lane_mask(bad) == 0ull;
    };
    const uint64_t t0 = wall_clock64();
    bool ok = false;
    look(u);
    for (;;) {
        __builtin_amdgcn_s_sleep(1);
        look(v);
        if (whole(u)) {
            ok = true;
            break;
        }
        if (wall_clock64() - t0 > wait) break;
        __builtin_amdgcn_s_sleep(1);
        look(u);
        if (whole(v)) {
#pragma unroll
            for (int k = 0; k < LY::KS; k++) u[k] = v[k];
            ok = true;
            break;
        }
        if (wall_clock64() - t0 > wait) break;
    }
    if (!ok) return false;
    leaf = __builtin_amdgcn_readlane((int)(uint32_t)(u[LW / 64] >> 32), LW % 64);
#pragma unroll
    for (int k = 0; k < LY::KS; k++) {
        const int w = 64 * k + lane;
        const uint32_t word = (uint32_t)(u[k] >> 32);
        if (w < S * N / 4) ((uint32_t *)qs)[w] = word;
        else if (w < LY::SW) ((uint32_t *)sp)[w - S * N / 4] = word;
    }
    wave_sync();
    return true;
}

// A step the stream computed itself: the states of layers 0 .. S - 1 after step t (LDS qs) into every copy of the
// slot of its input x (tag E0 + t), for step t + 1's helpers
template <class SH, int S>
__device__ __forceinline__ void spec_publish(const YggIO &io, int t, int x, const int8_t *qs, int lane) {
    using LY = SpecLayout<SH, S>;
    const uint32_t tag = io.spec_epoch + (uint32_t)t;
    uint64_t *const slot = io.spec + kSpecSlots + (size_t)x * kSpecSlotUnits;
#pragma unroll
    for (int k = 0; k < LY::KP; k++) {
        const int w = 64 * k + lane;
        if (w < LY::PW) {
            const uint64_t v = spec_unit(tag, ((const uint32_t *)qs)[w]);
#pragma unroll
            for (int c = 0; c < kSpecCopies; c++) spec_store(slot + c * kSpecCopyUnits + w, v);
        }
    }
}

// the stream's input x of step t, for step t's helpers (lane c stores copy c)
__device__ __forceinline__ void spec_token(const YggIO &io, int t, int x, int lane) {
    if (lane < kSpecCopies)
        spec_store(io.spec + kSpecTok + (size_t)lane * kSpecCopyUnits,
                   spec_unit(io.spec_epoch + (uint32_t)t, (uint32_t)x));
}

}  // namespace ygg
