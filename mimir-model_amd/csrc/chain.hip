// One launch for a chain of dependent one-row products: Q4_K / Q6_K weights
// x 8-bit activations in blocks of 256 (dequant_matmul_a8.v2, reference
// interp/fast.go:246-379), phase after phase, where a phase is the grouped
// call of 1..3 matrices on one input row (the q/k/v, o, gate/up and down
// calls importer/llama.go:423-534 writes) and a later phase may read what
// an earlier one wrote. The results are bit for bit those of the separate
// calls (same exact (S, M) per block, same float chain in block order as
// dotQ8KRef, internal/kernels/q8k_test.go:38-102; same quantizer,
// q8.go:50-97; same float32 path for refused rows, fast.go:323-377).
//
// Why one launch. At one activation row each product streams its weights
// once; the time between dependent launches (drain, launch, the first
// loads' round trip) is idle HBM. Here the weight bytes of every phase are
// streamed without a break: a workgroup per CU (all co-resident), whose
// copy waves fetch its share of each matrix (a contiguous byte range per
// matrix and phase, balanced by bytes) into an LDS ring with
// global_load_lds, up to NSLOT-1 stages ahead, across phase boundaries.
// The compute waves consume the ring; only they wait for a phase's input.
//
// Per workgroup: NCW compute waves and NCP copy waves. A stage is up to
// 16 KB: a run of whole rows of one matrix. Stage t sits in ring slot
// t % NSLOT. Every wave runs the same sequence of barriers:
//   B_t   stage t has landed (the copy waves waited for it) and slot
//         (t-1) % NSLOT is free; the copy waves then issue stage t+NSLOT-1
//   (first stage of a phase p > 0)
//   PE    thread 0 has seen phase p-1 complete on the device barrier
//   QD    the compute waves quantized phase p's input row into LDS
//   (last stage of a phase)
//   X     the phase's pairs are in the pair table; the compute waves then
//         run the float chains, add the bias, run the float32 path of
//         refused rows and store the outputs
//   Y     the phase's outputs are stored and acknowledged; thread 0 then
//         arrives at phase p's device barrier
// Compute waves: each group of eight lanes forms two (row, block) pairs'
// exact (S, M) from the ring with the decode GEMV's lane code
// (kquant_lane.hpp) into a pair table that holds the workgroup's whole
// phase ([row][block], at most CHAIN_TABLE_ENTRIES). The serial float
// chains (nb dependent fmas a row) run once per phase, every row at once,
// after its last stage (X): within a stage loop the waves only form pairs.
// Within a phase no wave touches global memory but through its copies: all
// global loads and stores of results wait for the phase's end (a wave's
// loads and stores retire in order on one counter, so a wait for one would
// wait for all).
//
// Device barrier between phases (two levels, so that no counter takes more
// than 16 of the launch's atomics): workgroup g counts in on line counter
// g % 16 (agent-scope atomic), the workgroup completing a line adds one to
// the phase's top counter, and every workgroup's thread 0 polls the top
// counter with agent-scope loads. Counters only grow: the line counter's old
// value tells the launch number e (floor(old / workgroups on the line)),
// and the top counter is complete at (e + 1) * 16; so the counters need no
// reset and a captured graph can be replayed. A buffer of counters serves
// launches that do not overlap in time on one device. Every poll is bounded:
// past POLL_LIMIT tries the workgroup sets the status word, stops waiting
// and finishes (its outputs are then not valid), so no launch can hang.
//
// Data between phases: outputs are stored with agent-scope stores (through
// the XCD's L2 to memory) and the phase input is read with agent-scope loads
// (past the L2), so a row written by another XCD's workgroup is seen once
// its phase's barrier has passed.
#include "f32path.hpp"
#include "kquant_lane.hpp"
#include "mimg_device.hpp"
#include "mimg_kernels.hpp"
#include "qa_chunk.hpp"

namespace mimg {
namespace chn {

constexpr int NCW = 8;                  // compute waves
constexpr int NCP = 4;                  // copy waves
constexpr int NTH = 64 * (NCW + NCP);   // threads per workgroup
constexpr int SB = CHAIN_STAGE_BYTES;   // bytes per ring slot (one stage)
constexpr int NSLOT = 6;
constexpr int IPW = SB / 1024 / NCP;    // copy instructions per stage and copy wave
constexpr int NGRP = NCW * 8;           // groups of eight lanes
constexpr int MAXPAIRS = CHAIN_MAX_PAIRS;
constexpr int LINES = CHAIN_LINES;
constexpr uint32_t POLL_LIMIT = 1u << 18;
static_assert(MAXPAIRS == 2 * NGRP, "two rounds of the groups per stage");

struct Smem {
    uint8_t ring[NSLOT * SB];
    int8_t q[CHAIN_MAXK];
    float d32[CHAIN_MAXK / 32];
    int16_t xs[CHAIN_MAXK / 32];
    int16_t ys16[CHAIN_MAXK / 16];
    i32x4 table[CHAIN_TABLE_ENTRIES];  // [row of the workgroup's phase rows][block]
    int wbad[NCW];
};

// Global -> LDS copy of 16 bytes a lane (lane i writes at lds + 16 i). Inline
// assembly, so that the compiler does not wait for the copies in flight; the
// copy waves wait for them explicitly (WAIT_VMCNT).
__device__ __forceinline__ void copy16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
#define CH_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

// A workgroup barrier that waits for nothing in flight (the copy waves'
// copies stay outstanding); each wave writes out the waits it needs.
__device__ __forceinline__ void bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ uint64_t* counter(uint64_t* sync, int c) { return sync + 16 * (1 + c); }

// A value every lane holds, made a scalar: the kernel arguments are then
// read with scalar loads. (A vector load here would make the copy waves
// wait for every copy they have in flight.)
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
    const int lo = __builtin_amdgcn_readfirstlane((int)(v & 0xFFFFFFFF)), hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// floor(a / b) for a < 2^53 and a small b: the double quotient, corrected.
__device__ __forceinline__ int64_t div_floor(int64_t a, int64_t b) {
    int64_t q = uni64((int64_t)((double)a / (double)b));
    while (q * b > a) q--;
    while ((q + 1) * b <= a) q++;
    return q;
}

// The first row of the phase's concatenated matrices that starts at or
// after byte b of their concatenated bytes.
__device__ int row_at(const ChainPhase& P, int64_t b) {
    int64_t start = 0;
    int base = 0;
    for (int i = 0; i < P.nmat; i++) {
        const int64_t rb = P.m[i].rb, end = start + (int64_t)P.m[i].N * rb;
        if (b <= end || i == P.nmat - 1) {
            const int64_t num = b > start ? b - start : 0;
            int64_t q = div_floor(num + rb - 1, rb);
            if (q > P.m[i].N) q = P.m[i].N;
            return base + (int)q;
        }
        start = end;
        base += P.m[i].N;
    }
    return base;
}

// One stage: rows [row, row + n) of matrix mi of phase p (n = 0: an empty
// stage, for a workgroup with no rows in the phase).
struct StageD {
    int p, mi, row, n;
    int lrow;    // the stage's first row among the workgroup's rows of the phase
    int r0, r1;  // the workgroup's rows of the phase (over its concatenated matrices)
    bool first, last;
};

// The workgroup's stages in order: its rows of each phase (a byte-balanced
// split of the phase's bytes over the G workgroups), in runs of at most
// rps rows of one matrix.
struct Walker {
    int p, r0, r, r1, t;
    __device__ void phase_rows(const ChainArgs& A, int g) {
        const ChainPhase& P = A.ph[uni(p)];
        r = uni(row_at(P, div_floor(P.bytes * g, A.G)));
        r1 = uni(row_at(P, div_floor(P.bytes * (g + 1), A.G)));
        r0 = r;
    }
    __device__ void start(const ChainArgs& A, int g) {
        p = 0;
        t = 0;
        phase_rows(A, g);
    }
    __device__ bool next(const ChainArgs& A, int g, StageD& s) {
        p = uni(p);
        r0 = uni(r0);
        r = uni(r);
        r1 = uni(r1);
        t = uni(t);
        if (p >= A.nphase) return false;
        const ChainPhase& P = A.ph[p];
        int mi = 0, base = 0;
        while (mi + 1 < P.nmat && r >= base + P.m[mi].N) {
            base += P.m[mi].N;
            mi++;
        }
        mi = uni(mi);
        base = uni(base);
        int n = 0;
        if (r < r1) n = min(P.m[mi].rps, min(r1 - r, base + P.m[mi].N - r));
        s.p = p;
        s.mi = uni(mi);
        s.row = uni(r - base);
        s.n = uni(n);
        s.lrow = r - r0;
        s.r0 = r0;
        s.r1 = r1;
        s.first = t == 0;
        r += n;
        t++;
        s.last = r >= r1;
        if (s.last) {
            p++;
            t = 0;
            if (p < A.nphase) phase_rows(A, g);
        }
        return true;
    }
};

// Copy wave cw's share of a stage into ring slot `slot` (IPW instructions of
// 1 KB; lanes past the stage's bytes reload its last 16, so every copy wave
// issues the same count per stage). s == null or an empty stage: a dummy
// copy of 16 bytes the chain's first matrix surely has.
__device__ __forceinline__ void issue_stage(const ChainArgs& A, const StageD& s, bool valid, int slot, int cw,
                                            int lane, uint32_t ring0) {
    const uint8_t* base = A.ph[0].m[0].W;
    int64_t bytes = 16;
    if (valid && s.n > 0) {
        const ChainMat& M = A.ph[uni(s.p)].m[uni(s.mi)];
        base = M.W + (int64_t)s.row * M.rb;
        bytes = (int64_t)s.n * M.rb;
    }
#pragma unroll
    for (int k = 0; k < IPW; k++) {
        const int qi = cw + NCP * k;
        int64_t off = (int64_t)qi * 1024 + 16 * lane;
        if (off > bytes - 16) off = bytes - 16;
        copy16(base + off, ring0 + (uint32_t)(slot * SB + qi * 1024));
    }
}

// Eight 16-byte loads of the input row with agent scope (sc1: past the
// XCD's L2, so a row another XCD's workgroup stored is seen), issued
// together and waited for inside the same statement (the compiler does not
// track loads written in assembly; the compute waves have nothing else in
// flight here).
__device__ __forceinline__ void load8_coh(const float* const* p, u32x4* v) {
    asm volatile(
        "global_load_dwordx4 %0, %8, off sc1\n\t"
        "global_load_dwordx4 %1, %9, off sc1\n\t"
        "global_load_dwordx4 %2, %10, off sc1\n\t"
        "global_load_dwordx4 %3, %11, off sc1\n\t"
        "global_load_dwordx4 %4, %12, off sc1\n\t"
        "global_load_dwordx4 %5, %13, off sc1\n\t"
        "global_load_dwordx4 %6, %14, off sc1\n\t"
        "global_load_dwordx4 %7, %15, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
        : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6]), "v"(p[7])
        : "memory");
}

// The phase's input row quantized into LDS (the quantizer launch's chunks:
// chunk c of 256 elements by compute wave c % NCW, four elements a lane);
// the wave's refusal flag goes to wbad[wave].
__device__ __forceinline__ void quantize_row(const ChainPhase& P, Smem& S, int wave, int lane) {
    constexpr int CPW = CHAIN_MAXK / 256 / NCW;
    static_assert(CPW == 8, "load8_coh loads eight chunks");
    const int K = P.K, nch = K / 256;
    const float* ptr[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) ptr[i] = P.x + 256 * min(wave + NCW * i, nch - 1) + 4 * lane;  // past the row: reloads
    u32x4 raw[CPW];
    load8_coh(ptr, raw);
    float4 v[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++)
        v[i] = make_float4(__uint_as_float(raw[i].x), __uint_as_float(raw[i].y), __uint_as_float(raw[i].z),
                           __uint_as_float(raw[i].w));
    ActPtrs a;
    a.q = S.q;
    a.d32 = S.d32;
    a.xs = S.xs;
    a.ys16 = S.ys16;
    a.dbs = nullptr;
    a.ok = nullptr;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int c = wave + NCW * i;
        if (c < nch) bad |= qa_chunk<256>(v[i], 0, (int64_t)256 * c + 4 * lane, K, a, lane);
    }
    if (lane == 0) S.wbad[wave] = bad ? 1 : 0;
}

__device__ __forceinline__ bool row_refused(const Smem& S) {
    int r = 0;
#pragma unroll
    for (int w = 0; w < NCW; w++) r |= S.wbad[w];
    return r != 0;
}

// The stage's (row, block) pairs, group grp (of NGRP) taking pairs grp,
// grp + NGRP: exact (S, M) and the two scale products into the table.
__device__ __forceinline__ void stage_pairs(const ChainArgs& A, const StageD& s, Smem& S, int slot, int grp,
                                            int l) {
    static_assert(MAXPAIRS == 2 * NGRP, "one round of two pairs a group");
    if (s.n == 0) return;
    const ChainPhase& P = A.ph[uni(s.p)];
    const ChainMat& M = P.m[uni(s.mi)];
    const int nb = P.nb, npairs = s.n * nb;
    if (grp >= npairs) return;
    const uint32_t inv = (65536u + (uint32_t)nb - 1) / (uint32_t)nb;  // j / nb for j < 2^16 / nb: (j * inv) >> 16
    const uint8_t* sl = S.ring + slot * SB;
    const int64_t K = P.K;
    // the group's two pairs, grp and grp + NGRP (the second clamped: its
    // loads are issued with the first's, its entry is stored only if real)
    const int j0 = grp, j1 = min(grp + NGRP, npairs - 1);
    const bool two = grp + NGRP < npairs;
    const int r0 = (int)(((uint32_t)j0 * inv) >> 16), b0 = j0 - r0 * nb;
    const int r1 = (int)(((uint32_t)j1 * inv) >> 16), b1 = j1 - r1 * nb;
    if (M.dt == DT_Q4_K) {
        const Q6KRaw none = {};
        const uint8_t* k0 = sl + r0 * M.rb + b0 * Q4K_BYTES;
        const uint8_t* k1 = sl + r1 * M.rb + b1 * Q4K_BYTES;
        const u32x4 h0 = *(const u32x4*)k0, q0 = *(const u32x4*)(k0 + 16 + 16 * l);
        const u32x4 h1 = *(const u32x4*)k1, q1 = *(const u32x4*)(k1 + 16 + 16 * l);
        const ActLane a0 = act_lane<DT_Q4_K>(S.q, S.xs, S.d32, K, 0, b0, l);
        const ActLane a1 = act_lane<DT_Q4_K>(S.q, S.xs, S.d32, K, 0, b1, l);
        const i32x4 v0 = pair_part<DT_Q4_K>(h0, q0, none, a0, l);
        const i32x4 v1 = pair_part<DT_Q4_K>(h1, q1, none, a1, l);
        if (l == 0) {
            S.table[s.lrow * nb + j0] = v0;
            if (two) S.table[s.lrow * nb + j1] = v1;
        }
    } else {
        const u32x4 z = {0u, 0u, 0u, 0u};
        const Q6KRaw w0 = q6k_load_at(sl, (uint32_t)(r0 * M.rb + b0 * Q6K_BYTES), l);
        const Q6KRaw w1 = q6k_load_at(sl, (uint32_t)(r1 * M.rb + b1 * Q6K_BYTES), l);
        const ActLane a0 = act_lane<DT_Q6_K>(S.q, S.ys16, S.d32, K, 0, b0, l);
        const ActLane a1 = act_lane<DT_Q6_K>(S.q, S.ys16, S.d32, K, 0, b1, l);
        const i32x4 v0 = pair_part<DT_Q6_K>(z, z, w0, a0, l);
        const i32x4 v1 = pair_part<DT_Q6_K>(z, z, w1, a1, l);
        if (l == 0) {
            S.table[s.lrow * nb + j0] = v0;
            if (two) S.table[s.lrow * nb + j1] = v1;
        }
    }
}

// A row's float chain over its table entries: the blocks in order, the
// entries of eight blocks read at once, then their fmas.
template <bool Q4K>
__device__ __forceinline__ float row_chain(const i32x4* tb, int nb) {
    constexpr int BATCH = 8;
    float tot = 0.f, off = 0.f;
    for (int b0 = 0; b0 < nb; b0 += BATCH) {
        int sv[BATCH], mv[Q4K ? BATCH : 1];
        float dv[BATCH], ov[Q4K ? BATCH : 1];
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
            const i32x4* e = tb + min(b0 + u, nb - 1);
            if constexpr (Q4K) {
                const i32x4 v = *e;
                sv[u] = v.x;
                mv[u] = v.y;
                dv[u] = __int_as_float(v.z);
                ov[u] = __int_as_float(v.w);
            } else {
                sv[u] = e->x;
                dv[u] = __int_as_float(e->z);
            }
        }
#pragma unroll
        for (int u = 0; u < BATCH; u++) {
            if (b0 + u < nb) {
                tot = __builtin_fmaf((float)sv[u], dv[u], tot);
                if constexpr (Q4K) off = __builtin_fmaf((float)mv[u], ov[u], off);
            }
        }
    }
    return Q4K ? tot - off : tot;
}

// The phase's outputs (the compute waves, after its last stage's pairs):
// every row's float chain at once (one lane a row, over the blocks in
// order), then y = the chain (+ bias), or, for rows the reference refuses
// (the input row, or a weight row with a non-finite block scale), the
// float32 path, a group of eight lanes a row. Stored with agent-scope
// stores. The whole phase's pairs stay in LDS until here, so the chains
// (serial, nb dependent fmas) run once per phase and not in the stage loop.
__device__ __forceinline__ void phase_outputs(const ChainArgs& A, const StageD& s, const Smem& S, bool actref,
                                              int tid) {
    const ChainPhase& P = A.ph[uni(s.p)];
    const int nb = P.nb;
    int base = 0;
    for (int mi = 0; mi < P.nmat; mi++) {
        const ChainMat& M = P.m[mi];
        const bool q4k = M.dt == DT_Q4_K;
        const int lo = max(s.r0, base), hi = min(s.r1, base + M.N);  // this matrix's rows of the workgroup
        for (int gr = lo + tid; gr < hi; gr += 64 * NCW) {
            const int row = gr - base;
            if (actref || (M.nref && M.wref[row])) continue;
            const i32x4* tb = S.table + (gr - s.r0) * nb;
            float v = q4k ? row_chain<true>(tb, nb) : row_chain<false>(tb, nb);
            if (M.bias) v += M.bias[row];
            __hip_atomic_store(M.y + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (actref || M.nref) {
            for (int gr = lo + (tid >> 3); gr < hi; gr += 8 * NCW) {
                const int row = gr - base;
                if (!actref && M.wref[row] == 0) continue;  // the same for the group's eight lanes
                const uint8_t* wrow = M.W + (int64_t)row * M.rb;
                float res = q4k ? f32dot_g8<DT_Q4_K, true>(wrow, P.x, P.K, true)
                                : f32dot_g8<DT_Q6_K, true>(wrow, P.x, P.K, true);
                if (M.bias) res += M.bias[row];
                if ((tid & 7) == 0) __hip_atomic_store(M.y + row, res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        base += M.N;
    }
}

// Phase p's device barrier, arrival side (thread 0): returns the top
// counter's value once the whole launch has arrived.
__device__ __forceinline__ uint64_t arrive(const ChainArgs& A, int p, int g) {
    const int line = g % A.lines;
    const int64_t per = (A.G - line + A.lines - 1) / A.lines;
    const int c0 = p * (LINES + 1);
    const uint64_t o = __hip_atomic_fetch_add(counter(A.sync, c0 + 1 + line), (uint64_t)1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    const int64_t e = div_floor((int64_t)o, per);
    if ((int64_t)o == (e + 1) * per - 1)
        __hip_atomic_fetch_add(counter(A.sync, c0), (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (uint64_t)(e + 1) * (uint64_t)A.lines;
}

// Waiting side (thread 0): false after POLL_LIMIT tries (status word set).
__device__ __forceinline__ bool wait_phase(const ChainArgs& A, int p, uint64_t want) {
    const uint64_t* top = counter(A.sync, p * (LINES + 1));
    for (uint32_t it = 0; it < POLL_LIMIT; it++) {
        if (__hip_atomic_load(top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= want) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    __hip_atomic_store((uint32_t*)A.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

// The copy waves: the ring's producer. They take every barrier the compute
// waves take (same walker, same stages) and issue nothing the compiler
// tracks, so no wait of theirs covers more than the stage they wait for.
__device__ __forceinline__ void copy_waves(const ChainArgs& A, int g, int cw, int lane, uint32_t ring0) {
    Walker ahead, cur;
    ahead.start(A, g);
    cur.start(A, g);
    auto issue = [&](int slot) {
        StageD a;
        const bool ok = ahead.next(A, g, a);
        issue_stage(A, a, ok, slot, cw, lane, ring0);
    };
    for (int t = 0; t < NSLOT - 1; t++) issue(t);  // the first NSLOT-1 stages, before anything waits
    bar();  // the phase-0 row is in LDS
    StageD s;
    for (int t = 0; cur.next(A, g, s); t++) {
        CH_WAIT_VMCNT(IPW * (NSLOT - 2));  // stage t has landed
        bar();                             // B_t
        issue((t + NSLOT - 1) % NSLOT);
        if (s.first && s.p > 0) {
            bar();  // PE
            bar();  // QD
        }
        if (s.last) {
            bar();  // X
            bar();  // Y
        }
    }
    CH_WAIT_VMCNT(0);
}

// The compute waves: quantize each phase's row, form the pairs, run the
// chains, and (thread 0) the device barrier between phases.
__device__ __forceinline__ void compute_waves(const ChainArgs& A, Smem& S, int g, int wave, int lane) {
    quantize_row(A.ph[0], S, wave, lane);  // phase 0's input needs no wait
    bar();                                 // the phase-0 row is in LDS
    bool actref = row_refused(S);
    Walker cur;
    cur.start(A, g);
    StageD s;
    bool dead = false;
    uint64_t want = 0;
    for (int t = 0; cur.next(A, g, s); t++) {
        bar();  // B_t
        if (s.first && s.p > 0) {
            if (threadIdx.x == 0 && !dead) dead = !wait_phase(A, s.p - 1, want);
            bar();  // PE
            quantize_row(A.ph[uni(s.p)], S, wave, lane);
            bar();  // QD
            actref = row_refused(S);
        }
        stage_pairs(A, s, S, t % NSLOT, wave * 8 + (lane >> 3), lane & 7);
        if (s.last) {
            bar();  // X: the phase's pairs are all in the table
            phase_outputs(A, s, S, actref, threadIdx.x);
            CH_WAIT_VMCNT(0);  // the outputs are acknowledged
            bar();             // Y
            if (threadIdx.x == 0 && s.p < A.nphase - 1) want = arrive(A, s.p, g);
        }
    }
}

__global__ __launch_bounds__(NTH) void chain_kernel(ChainArgs A) {
    __shared__ __align__(16) Smem S;
    const int g = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave >= NCW)
        copy_waves(A, g, wave - NCW, lane, __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)S.ring));
    else
        compute_waves(A, S, g, wave, lane);
}

}  // namespace chn

__global__ void chain_zero_kernel(uint64_t* p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

hipError_t launch_chain_zero(void* p, uint64_t bytes, hipStream_t stream) {
    hipLaunchKernelGGL(chain_zero_kernel, dim3(8), dim3(256), 0, stream, (uint64_t*)p, (int64_t)(bytes / 8));
    return hipGetLastError();
}

int chain_occupancy() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, chn::chain_kernel, chn::NTH, 0) != hipSuccess) return 0;
    return n;
}

hipError_t launch_chain(const ChainArgs& A, hipStream_t stream) {
    hipLaunchKernelGGL(chn::chain_kernel, dim3((unsigned)A.G), dim3(chn::NTH), 0, stream, A);
    return hipGetLastError();
}

}  // namespace mimg
