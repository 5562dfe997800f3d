// step.h - the whole decode step as ONE persistent kernel (k_step).
//
// The per-op graph (engine.hip) runs a decode step as 161 kernels; each
// GEMV pays a kernel boundary, the wait for its inputs, its prologue and its
// fold tail before its weight stream reaches full rate, about as long as
// the stream itself at the 7B shape.  k_step keeps the weight stream going
// across those boundaries:
//
//   * one workgroup per CU (the grid is the CU count, every workgroup
//     resident), 7 compute waves + 1 control wave (two waves per SIMD, so
//     that a wave may hold 256 registers);
//   * the step's phases run in order - per layer QKV, attention, wo, w1|w3,
//     w2, then the classifier - separated by a grid barrier (grid_sync);
//   * a GEMV phase deals row pairs to workgroups (pair b, b + grid, ...) and
//     the (row, 1 KiB sweep) items of a workgroup's rows round-robin to its
//     compute waves, so every wave of the grid has the same number of items
//     (+-1); the terms of every group go to a workgroup fold area, and after
//     the items one lane per row folds them in group order;
//   * every compute wave streams its items through a ring of three register
//     slots of four items (four 16-byte weight loads + four scale dwords):
//     while it consumes one slot the next two are in flight, and the ring
//     runs on from one phase into the next (the next phase's first items are
//     loaded while the barrier and the prologue of that phase run).  The ring
//     does not cross an attention phase (the attention's K/V loads would
//     queue behind the weights): there it holds loads of a fixed cached
//     line, and the real items are issued when the attention is done;
//   * the control wave runs the barrier, persists the residual stream and
//     stores the outputs the compute waves staged in LDS, so the compute
//     waves never wait for a store or a barrier poll behind their ring.
//
// The arithmetic is the per-op kernels', operation for operation (the same
// group dots, the ordered fold, the RMSNorm chain in the reference's 16-lane
// order, the host-identical expf, the host-built RoPE table and the exact
// attention), so the step is bit-identical to them and to runq.c.
//
// Shapes (template parameters D = dim, H = hidden, HS = head size): INT4
// weights in groups of 64; rows of the dim-wide GEMVs (qkv, wo, w1|w3,
// classifier) are 2 sweeps of 1 KiB (1024 < D/2 <= 2048), rows of w2 are 5
// or 6 sweeps (4096 < H/2 <= 6144).  The engine instantiates the Llama-2-7B
// shape (4096, 11008, 128); other shapes run the per-op graph.
#pragma once
#include <type_traits>

#include "gemv.h"
#include "kernels.h"
#include "step_args.h"

namespace l2q {

static_assert(kVDims == kStepAttnSlice, "attention slice");

constexpr int kStepSlack = 32;       // floats after the fold area (fold_row reads ahead)
constexpr int kStepMaxT = 4096;      // cache positions the attention area holds
constexpr int kStepItems = 4;        // items per ring slot
constexpr int kStepMaxPairs = kStepPairsCap;    // row pairs of a dim-wide GEMV per workgroup (classifier: 16000 / 256)
constexpr int kStepMaxPairsH = kStepPairsCapH;  // row pairs of w2 per workgroup (2048 / 256)
constexpr unsigned long long kStepTimeout = 20000000ull;   // 200 ms of s_memrealtime (100 MHz)
// attention with the compute waves: one position per thread per round, V in
// chunks of one position per thread
constexpr int kSAThreads = kStepCThreads;
constexpr int kSAChunk = kSAThreads;
constexpr int kSAStride = kSAChunk + 4;
constexpr int kSAVPer = kSAChunk * kStepAttnSlice / 4 / kSAThreads;
constexpr int kSARounds = (kStepMaxT + kSAThreads - 1) / kSAThreads;

enum StepKind : int { kSQkv = 0, kSAtt = 1, kSWo = 2, kSW13 = 3, kSW2 = 4, kSCls = 5 };
__device__ __forceinline__ int phase_kind(int p, int L) { return p >= 5 * L ? kSCls : p % 5; }

#ifdef L2Q_STEP_TRACE
// diagnostic build only: s_memrealtime stamps [workgroup][phase][8]
__device__ unsigned long long g_step_trace[256 * 1024 * 8];
#define STEP_TRACE(p, k)                                                                          \
    do {                                                                                          \
        if ((threadIdx.x & 63) == 0)                                                              \
            g_step_trace[((size_t)blockIdx.x * 1024 + (p)) * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define STEP_TRACE(p, k) \
    do {                 \
    } while (0)
#endif

__host__ __device__ constexpr int r4(int v) { return (v + 3) / 4 * 4; }

// Geometry of one GEMV kind: rows of NS weight sweeps and NSS scale sweeps;
// item s of a row carries scale sweep s / (NS / NSS) when s is a multiple of
// NS / NSS.
template <int D, int H, int KIND>
struct GemvKind {
    static constexpr bool B = KIND == kSW2;
    static constexpr int COLS = B ? H : D;
    static constexpr int ROWB = COLS / 2;
    static constexpr int NS = (ROWB + kSweepBytes - 1) / kSweepBytes;
    static constexpr int NB = COLS / 64;
    static constexpr int NSS = (NB + L2Q_WAVE - 1) / L2Q_WAVE;
    static constexpr int SEVERY = NS / NSS;
    static_assert(NS % NSS == 0, "scale sweeps ride on weight sweeps");
    static constexpr int NBP = gemv_nbp(NB);
};

// Compile-time LDS layout (floats) of k_step<D, H, HS>.
template <int D, int H, int HS>
struct StepShape {
    static_assert(D % 64 == 0 && H % 64 == 0, "groups of 64");
    static_assert(D / 2 > kSweepBytes && D / 2 <= 2 * kSweepBytes, "dim rows of two sweeps");
    static_assert(H / 2 > 4 * kSweepBytes && H / 2 <= 6 * kSweepBytes, "hidden rows of five or six sweeps");
    static constexpr int kDH = D > H ? D : H;
    // shared
    static constexpr int kMisc = 0;   // [0] inv, [1] abort, [2] token, [3] pos, [8..72) exp table
    static constexpr int kCnt = kMisc + 72;
    static constexpr int kStOff = kCnt + 8;
    static constexpr int kStVal = kStOff + kStepCompute * kStepStage;
    static constexpr int kUni = r4(kStVal + kStepCompute * kStepStage);
    // GEMV phase
    static constexpr int kIn0 = kUni;                 // v = x + resid of a norm phase (residual persist)
    static constexpr int kRope = kIn0 + r4(D);        // the position's RoPE row
    static constexpr int kVs = kRope + r4(HS);
    static constexpr int kAct = kVs + 16 * ((D / 16 + 3) / 4 * 4 + 4);   // sumsq_stride(D)
    static constexpr int kActS = kAct + r4((kDH + 31) / 32 * 32 / 4);
    static constexpr int kFold = kActS + r4(kDH / 64);
    // fold area: [rows][nbp] terms, then [rows][nbp] scales
    static constexpr int kFoldD = 2 * (2 * kStepMaxPairs) * GemvKind<D, H, kSQkv>::NBP;
    static constexpr int kFoldH = 2 * (2 * kStepMaxPairsH) * GemvKind<D, H, kSW2>::NBP;
    static constexpr int kGemvEnd = kFold + (kFoldD > kFoldH ? kFoldD : kFoldH) + kStepSlack;
    // attention phase
    static constexpr int kAq = kUni;
    static constexpr int kAp = kAq + r4(HS);
    static constexpr int kAvt = kAp + kStepMaxT + kRingSlack;
    static constexpr int kAred = kAvt + 2 * kVDims * kSAStride + kRingSlack;
    static constexpr int kAttEnd = kAred + 16;
    static constexpr int kTotal = kGemvEnd > kAttEnd ? kGemvEnd : kAttEnd;
};

// Workgroup barrier that orders LDS only: its fences are scoped to LDS, so
// the hardware waits for this wave's LDS operations (lgkmcnt) and never for
// its loads in flight; the empty asm statements keep the compiler from
// moving any memory access across it.
__device__ __forceinline__ void wg_bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------
// Grid barrier (control wave): workgroups arrive on the counter of their
// group (blockIdx % 8: one XCD each); the last arrival of a group bumps the
// top counter, and the last group's last arrival writes every workgroup's
// release word, which each workgroup polls on its own line.  Barrier k of
// launch e waits for the value e * nbar + k (32-bit arithmetic wraps
// consistently, comparisons are on differences), so no state is reset
// between launches.  Every wait is bounded: past kStepTimeout the error word
// is set and every workgroup returns false from its next wait.
__device__ __forceinline__ bool grid_sync(const StepSync& s, unsigned k, int lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");   // this workgroup's stores, to memory
    const unsigned ng = 8, per = gridDim.x / ng;
    int last = 0;
    if (lane == 0) {
        const unsigned old = __hip_atomic_fetch_add(s.grp + 16 * (blockIdx.x % ng), 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (old == k * per - 1)
            last = __hip_atomic_fetch_add(s.top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == k * ng - 1;
    }
    last = __shfl(last, 0);
    if (last)
        for (unsigned i = lane; i < gridDim.x; i += L2Q_WAVE)
            __hip_atomic_store(s.rel + 16 * i, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int ok = 1;
    if (lane == 0) {
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        const unsigned* mine = s.rel + 16 * blockIdx.x;
        while ((int)(__hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - k) < 0) {
            if (__hip_atomic_load(s.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) { ok = 0; break; }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kStepTimeout) {
                __hip_atomic_fetch_or(s.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
        }
    }
    ok = __shfl(ok, 0);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // what other workgroups stored, visible here
    return ok;
}

// Staged outputs of a wave: (base << 30 | element offset, value) pairs,
// appended in lane order; base 0 = the phase's output vector, 1 = the
// layer's K cache, 2 = its V cache.
struct Stager {
    unsigned* off;
    float* val;
    int n;
    __device__ __forceinline__ void put(bool valid, unsigned o, float v) {
        const unsigned long long m = __ballot(valid);
        const int idx = __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0));
        if (valid) {
            off[n + idx] = o;
            val[n + idx] = v;
        }
        n += __popcll(m);
    }
};

template <int V>
using IC = std::integral_constant<int, V>;

// The lane index through an empty asm statement: values derived from it
// inside a phase cannot be hoisted out of the step's phase loop (where they
// would stay live, each in a register, through every other phase).
__device__ __forceinline__ int opaque_lane(int lane) {
    asm volatile("" : "+v"(lane));
    return lane;
}
// A wave-uniform value the compiler cannot see through (keeps the ordered
// fold a loop instead of a full unroll whose hoisted LDS reads would need a
// register each).
__device__ __forceinline__ int opaque_uniform(int v) {
    asm volatile("" : "+s"(v));
    return v;
}
constexpr unsigned kVmcnt0 = 0x0F70;   // s_waitcnt vmcnt(0)

// ---------------------------------------------------------------------------
// Register ring of GEMV items.

struct Slot {
    uint4 w[kStepItems];
    float s[kStepItems];
};

// Rows and weights of the GEMV of phase p.
struct PhaseW {
    int kind, rows;
    const uint8_t* w;
    const float* ws;
};

template <int D, int H>
__device__ __forceinline__ PhaseW phase_w(const StepArgs& a, int p) {
    PhaseW g;
    const int P = step_phases(a.L);
    g.kind = p < P ? phase_kind(p, a.L) : kSAtt;
    const int l = p / 5, qkv_rows = D + 2 * a.kv;
    constexpr int RD = D / 2, RH = H / 2, ND = D / 64, NH = H / 64;
    switch (g.kind) {
        case kSQkv:
            g.rows = qkv_rows;
            g.w = a.qkv_w + (size_t)l * qkv_rows * RD; g.ws = a.qkv_s + (size_t)l * qkv_rows * ND;
            break;
        case kSWo:
            g.rows = D;
            g.w = a.wo_w + (size_t)l * D * RD; g.ws = a.wo_s + (size_t)l * D * ND;
            break;
        case kSW13:
            g.rows = 2 * H;
            g.w = a.w13_w + (size_t)l * 2 * H * RD; g.ws = a.w13_s + (size_t)l * 2 * H * ND;
            break;
        case kSW2:
            g.rows = D;
            g.w = a.w2_w + (size_t)l * D * RH; g.ws = a.w2_s + (size_t)l * D * NH;
            break;
        case kSCls:
            g.rows = a.V;
            g.w = a.wcls_w; g.ws = a.wcls_s;
            break;
        default:   // attention, or past the last phase: no items
            g.rows = 0;
            g.w = a.wcls_w; g.ws = a.wcls_s;
            break;
    }
    return g;
}

// Items of phase p held by compute wave wv of this workgroup: the workgroup
// takes row pairs b, b + grid, ...; item i = r * NS + s of its rows (local
// row r, sweep s) goes to wave i % kStepCompute.
__device__ __forceinline__ int wg_rows(int rows) {
    const int npairs = (rows + 1) / 2;
    const int b = blockIdx.x;
    return b < npairs ? 2 * ((npairs - b + (int)gridDim.x - 1) / (int)gridDim.x) : 0;
}
__device__ __forceinline__ int wave_items(int rows, int ns, int wv) {
    const int n = wg_rows(rows) * ns;
    return wv < n ? (n - wv + kStepCompute - 1) / kStepCompute : 0;
}
// global row of local row r
__device__ __forceinline__ int wg_row(int r) { return 2 * ((int)blockIdx.x + (r >> 1) * (int)gridDim.x) + (r & 1); }

// A wave's position in its item stream: phase p, slot j of its items of
// that phase (items 4j .. 4j+3 of the wave), the phase's weights.
struct Cursor {
    int p, j, nslots, ns;
    PhaseW g;
};

template <int D, int H>
__device__ __forceinline__ void cursor_enter(const StepArgs& a, Cursor& c, int p, int wv) {
    c.p = p;
    c.j = 0;
    c.g = phase_w<D, H>(a, p);
    c.ns = c.g.kind == kSW2 ? GemvKind<D, H, kSW2>::NS : GemvKind<D, H, kSQkv>::NS;
    c.nslots = (wave_items(c.g.rows, c.ns, wv) + kStepItems - 1) / kStepItems;
}

// Move to the first phase, from c.p on, in which this wave has items.
template <int D, int H>
__device__ __forceinline__ void cursor_skip(const StepArgs& a, Cursor& c, int wv) {
    const int P = step_phases(a.L);
    while (c.p < P && c.j >= c.nslots) cursor_enter<D, H>(a, c, c.p + 1, wv);
}

// Weight chunk and scale chunk of item i of the wave (clamped to valid
// addresses past the wave's items: those are never consumed).
template <int D, int H, int KIND>
__device__ __forceinline__ void item_load(const PhaseW& g, int wv, int i, int lane, uint4& w, float& sc) {
    using K = GemvKind<D, H, KIND>;
    const int li = wv + kStepCompute * i;            // item index in the workgroup
    const int r = li / K::NS, s = li - r * K::NS;
    const int row = min(wg_row(r), g.rows - 1);
    const int off = min(s * kSweepBytes + 16 * lane, K::ROWB - 16);
    w = load_stream(g.w + (size_t)row * K::ROWB + off);
    const int ss = s / K::SEVERY;
    sc = g.ws[(size_t)row * K::NB + min(ss * L2Q_WAVE + lane, K::NB - 1)];
}

// Load slot j of cursor c's phase into S, or (a held or past-the-end slot)
// a line that stays cached: eight loads either way.
template <int D, int H>
__device__ __forceinline__ void issue(const StepArgs& a, Slot& S, Cursor& c, int next_att, int wv, int lane) {
    const int P = step_phases(a.L);
    if (c.p >= P || c.p > next_att) {
        const uint4* d = reinterpret_cast<const uint4*>(a.wcls_w) + lane;
#pragma unroll
        for (int k = 0; k < kStepItems; k++) {
            S.w[k] = load_stream(d);
            S.s[k] = a.wcls_s[lane];
        }
        return;
    }
    if (c.g.kind == kSW2) {
#pragma unroll
        for (int k = 0; k < kStepItems; k++) item_load<D, H, kSW2>(c.g, wv, kStepItems * c.j + k, lane, S.w[k], S.s[k]);
    } else {
#pragma unroll
        for (int k = 0; k < kStepItems; k++) item_load<D, H, kSQkv>(c.g, wv, kStepItems * c.j + k, lane, S.w[k], S.s[k]);
    }
    c.j++;
    cursor_skip<D, H>(a, c, wv);
}

// ---------------------------------------------------------------------------
// Prologue (compute waves): load the phase input (v = x + resid for a norm
// phase, x_in = emb[token] at layer 0; the vector to quantize otherwise) and
// quantize it (after the RMSNorm for a norm phase) to act_q / act_s; the
// same operations as prologue_compute (gemv.h).  A norm phase leaves v in
// LDS (in0) for the control wave, which persists the residual stream.
// Workgroup barriers without a memory fence, mirrored by the control wave
// (kNorm: 3, kQuant: 1).
template <int PRO, int N>
__device__ __forceinline__ void step_prologue(const float* src, const float* res, const float* nw, float* in0,
                                              int8_t* act_q, float* act_s, float* vs, float* misc, int tid) {
#pragma clang fp contract(off)
    constexpr int G = 64;
    constexpr int nchunks = N / 4;
    constexpr int KC = (nchunks + kStepCThreads - 1) / kStepCThreads;
    const int lane = tid & (L2Q_WAVE - 1);
    float4 v[KC], w[KC];
#pragma unroll
    for (int k = 0; k < KC; k++) {
        const int c = min(tid + kStepCThreads * k, nchunks - 1);
        v[k] = reinterpret_cast<const float4*>(src)[c];
        if constexpr (PRO == kNorm) {
            const float4 r = reinterpret_cast<const float4*>(res ? res : src)[c];
            w[k] = reinterpret_cast<const float4*>(nw)[c];
            if (res) { v[k].x += r.x; v[k].y += r.y; v[k].z += r.z; v[k].w += r.w; }
        }
    }
    float inv = 1.0f;
    if constexpr (PRO == kNorm) {
        constexpr int st = sumsq_stride(N);
#pragma unroll
        for (int k = 0; k < KC; k++) {
            const int c = tid + kStepCThreads * k;
            if (c < nchunks) {
                const int e = 4 * c;
                vs[((e + 0) & 15) * st + (e >> 4)] = v[k].x;
                vs[((e + 1) & 15) * st + (e >> 4)] = v[k].y;
                vs[((e + 2) & 15) * st + (e >> 4)] = v[k].z;
                vs[((e + 3) & 15) * st + (e >> 4)] = v[k].w;
                reinterpret_cast<float4*>(in0)[c] = v[k];
            }
        }
        wg_bar();
        if (tid < L2Q_WAVE) {
            const float ss = runq_sumsq_t(vs, N, st, lane);
            if (lane == 0) misc[0] = 1.0f / sqrtf(ss / (float)N + 1e-5f);
        }
        wg_bar();
        inv = misc[0];
    }
    // a group of 64 is 16 consecutive threads of one wave; threads past the
    // vector join the group reductions with zeros
#pragma unroll
    for (int k = 0; k < KC; k++) {
        const int c = tid + kStepCThreads * k;
        const bool in = c < nchunks;
        float4 o = v[k];
        if constexpr (PRO == kNorm) {
            o.x = w[k].x * (inv * o.x); o.y = w[k].y * (inv * o.y);
            o.z = w[k].z * (inv * o.z); o.w = w[k].w * (inv * o.w);
        }
        if (!in) o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        unsigned mb = max(max(__float_as_uint(o.x) & 0x7fffffffu, __float_as_uint(o.y) & 0x7fffffffu),
                          max(__float_as_uint(o.z) & 0x7fffffffu, __float_as_uint(o.w) & 0x7fffffffu));
        mb = group_umax<G / 4>(mb);
        const float s = q8_scale(__uint_as_float(mb));
        const float r = q8_recip(s);
        if (in) {
            const unsigned b0 = q8_byte_fast(o.x, s, r), b1 = q8_byte_fast(o.y, s, r);
            const unsigned b2 = q8_byte_fast(o.z, s, r), b3 = q8_byte_fast(o.w, s, r);
            constexpr unsigned kLoBytes = 0x0c0c0400u;
            *reinterpret_cast<uint16_t*>(act_q + act_split_addr(4 * c)) = (uint16_t)__builtin_amdgcn_perm(b2, b0, kLoBytes);
            *reinterpret_cast<uint16_t*>(act_q + act_split_addr(4 * c + 1)) = (uint16_t)__builtin_amdgcn_perm(b3, b1, kLoBytes);
            if ((c % (G / 4)) == 0) act_s[c / (G / 4)] = s;
        }
    }
    wg_bar();
}

// ---------------------------------------------------------------------------
// One GEMV phase (compute waves): prologue, the wave's items through the
// ring (group terms and scales into the workgroup fold area), a workgroup
// barrier (mirrored by the control wave), the ordered fold with one lane per
// row and the epilogue into the stager.  C counts the slots this wave has
// consumed since the launch (slot C sits in ring register set C % 3).
template <int D, int H, int HS, int KIND>
__device__ __forceinline__ void gemv_phase(const StepArgs& a, int p, Slot (&ring)[3], int& C, Cursor& cur,
                                           int next_att, float* L, int wv, int lane, Stager& st) {
    using Sh = StepShape<D, H, HS>;
    using K = GemvKind<D, H, KIND>;
    lane = opaque_lane(lane);
    constexpr int PRO = (KIND == kSWo || KIND == kSW2) ? kQuant : kNorm;
    const int tid = wv * L2Q_WAVE + lane;
    const int l = p / 5;
    float* misc = L + Sh::kMisc;
    int8_t* act_q = reinterpret_cast<int8_t*>(L + Sh::kAct);
    float* act_s = L + Sh::kActS;
    const int pos = __float_as_int(misc[3]);

    // prologue inputs
    const float* src;
    const float* res = nullptr;
    const float* nw = nullptr;
    switch (KIND) {
        case kSQkv:
            src = l == 0 ? a.emb + (size_t)__float_as_int(misc[2]) * D : a.xa;
            res = l == 0 ? nullptr : a.ffn_out;
            nw = a.rms_att + (size_t)l * D;
            break;
        case kSWo: src = a.att; break;
        case kSW13: src = a.xb; res = a.wo_out; nw = a.rms_ffn + (size_t)l * D; break;
        case kSW2: src = a.hb; break;
        default: src = a.xa; res = a.ffn_out; nw = a.rms_final; break;
    }
    if (KIND == kSQkv && tid < HS) L[Sh::kRope + tid] = a.rope[(size_t)pos * HS + tid];
    step_prologue<PRO, K::COLS>(src, res, nw, L + Sh::kIn0, act_q, act_s, L + Sh::kVs, misc, tid);
    if (wv == 0) STEP_TRACE(p, 4);

    const int rows = KIND == kSQkv ? D + 2 * a.kv : KIND == kSWo ? D : KIND == kSW13 ? 2 * H : KIND == kSW2 ? D : a.V;
    const int nrows = wg_rows(rows);
    const int n = wave_items(rows, K::NS, wv);
    const int nslots = (n + kStepItems - 1) / kStepItems;
    constexpr int ROWCAP = 2 * (K::B ? kStepMaxPairsH : kStepMaxPairs);
    float* tb = L + Sh::kFold;                          // [row][NBP] terms
    float* sb = tb + ROWCAP * K::NBP;                   // [row][NBP] scales
    const bool leader = (lane & 1) == 0;                // two lanes per group of 64 INT4 weights
    const float* rope = L + Sh::kRope;
    const uint64_t* etab = reinterpret_cast<const uint64_t*>(misc + 8);

    // the per-sweep scale, bias term and group sum of this lane's activation chunk
    LaneActs<4, 64, K::NS, false> A;
    lane_scalars_lds<4, 64, K::NS>(A, act_q, act_s, K::COLS, lane);

    // item i of this wave: weight chunk w, scale chunk sc
    auto consume = [&](int i, const uint4 w, float sc) {
        const int li = wv + kStepCompute * i;
        const int r = li / K::NS, s = li - r * K::NS;
        int x[8];
        lds_chunk<4>(act_q, min((s * kSweepBytes + 16 * lane) * 2, K::COLS - 32), x);
        const int dp = chunk_dot_x<4>(w, x);
        const int d = group_isum<2>(dp) >> 4;   // exact: the x16 dot is a multiple of 16
        const int off = s * kSweepBytes + 16 * lane;
        // the lane's chunk scalars for sweep s (s is wave-uniform: a select over the sweeps)
        float xs = A.xs[0], xt = A.xt[0];
        int sq = A.sq[0];
#pragma unroll
        for (int k = 1; k < K::NS; k++)
            if (s == k) { xs = A.xs[k]; xt = A.xt[k]; sq = A.sq[k]; }
        if (leader && off < K::ROWB) tb[r * K::NBP + off / 32] = group_term(xs, xt, d, sq);
        if (s % K::SEVERY == 0) {
            const int gi = (s / K::SEVERY) * L2Q_WAVE + lane;
            if (gi < K::NB) sb[r * K::NBP + gi] = sc;
        }
    };
    auto step = [&](auto S, int j) {
        Slot& R = ring[S.value];
#pragma unroll
        for (int k = 0; k < kStepItems; k++)
            if (kStepItems * j + k < n) consume(kStepItems * j + k, R.w[k], R.s[k]);
        // the slot is free again: the slot three ahead streams in
        issue<D, H>(a, R, cur, next_att, wv, lane);
    };
    auto run = [&](auto s0, auto s1, auto s2) {
        for (int j = 0; j < nslots;) {
            step(s0, j);
            if (++j >= nslots) break;
            step(s1, j);
            if (++j >= nslots) break;
            step(s2, j);
            ++j;
        }
    };
    // every slot issued before this phase has landed by now (it was issued
    // before the barrier and the prologue): one full wait here lets the
    // compiler track the ring exactly from here on
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    switch (C % 3) {
        case 0: run(IC<0>{}, IC<1>{}, IC<2>{}); break;
        case 1: run(IC<1>{}, IC<2>{}, IC<0>{}); break;
        default: run(IC<2>{}, IC<0>{}, IC<1>{}); break;
    }
    C += nslots;
    if (wv == 0) STEP_TRACE(p, 5);
    wg_bar();   // every term of the workgroup's rows is in the fold area

    // ordered fold: row pair q of the workgroup on lanes (2k, 2k+1) of wave
    // q % 7, k = q / 7
    const int q = (lane >> 1) * kStepCompute + wv;
    const int r = 2 * q + (lane & 1);
    float sum = 0.0f;
    if (r < nrows) sum = fold_row<3>(tb + r * K::NBP, sb + r * K::NBP, opaque_uniform(K::NB));
    const int row = wg_row(r);
    const bool mine = r < nrows && row < rows;
    if constexpr (KIND == kSQkv) {
        // (even, odd) rows on lanes (2k, 2k+1): RoPE of q and k, append k and v
        const float other = dpp_f<kDppXor1>(sum);
        const int e = row < D ? row : row - D;
        const int eg = e / HS;
        const int hd = (e & ~1) - eg * HS;
        const float c = rope[min(hd, HS - 2)], sn = rope[min(hd, HS - 2) + 1];
        const bool odd = row & 1;
        const float v0 = odd ? other : sum, v1 = odd ? sum : other;
        const float rot = odd ? __builtin_fmaf(v0, sn, v1 * c) : __builtin_fmaf(v0, c, -(v1 * sn));
        unsigned o;
        float val = rot;
        if (row < D) {
            o = (unsigned)row;
        } else if (row < D + a.kv) {
            o = (1u << 30) | (unsigned)k_index(1, eg, pos, e - eg * HS, HS, a.max_t);
        } else {
            const int ev = row - D - a.kv;
            const int gv = ev / HS;
            o = (2u << 30) | (unsigned)(((size_t)gv * a.max_t + pos) * HS + (ev - gv * HS));
            val = sum;
        }
        st.put(mine, o, val);
    } else if constexpr (KIND == kSW13) {
#pragma clang fp contract(off)
        const float h3 = dpp_f<kDppXor1>(sum);
        float hv = sum;
        hv *= (1.0f / (1.0f + exp_runq_t(-hv, etab)));
        st.put(mine && (lane & 1) == 0, (unsigned)(row >> 1), hv * h3);
    } else {
        st.put(mine, (unsigned)row, sum);
    }
}

// ---------------------------------------------------------------------------
// Attention phase (compute waves): k_attn_fused's operations (kernels.h) for
// the (head, output slice) items of this workgroup, items it = blockIdx.x +
// k * gridDim.x, with 448 threads (rounds and V chunks of 448 positions:
// the same operations in the same order); 5 + nchunks workgroup barriers
// per item, mirrored by the control wave.
__device__ __forceinline__ int attn_items(const StepArgs& a) {
    const int items = a.n_heads * (a.hs / kVDims);
    return (int)blockIdx.x < items ? (items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
}

template <int D, int H, int HS>
__device__ __forceinline__ void attn_phase(const StepArgs& a, int l, float* L, int wv, int lane, Stager& st) {
#pragma clang fp contract(off)
    using Sh = StepShape<D, H, HS>;
    lane = opaque_lane(lane);
    constexpr int F4 = HS / 4;
    const int tid = wv * L2Q_WAVE + lane;
    float* misc = L + Sh::kMisc;
    float* qs = L + Sh::kAq;
    float* p = L + Sh::kAp;
    float* vt = L + Sh::kAvt;
    float* red = L + Sh::kAred;
    const uint64_t* etab = reinterpret_cast<const uint64_t*>(misc + 8);
    const int n = __float_as_int(misc[3]) + 1;
    const int max_t = a.max_t;
    const int kv_mul = a.n_heads / a.n_kv;
    const int nchunks = (n + kSAChunk - 1) / kSAChunk;
    const float* kc = a.kcache + (size_t)l * a.kv * max_t;
    const float* vc = a.vcache + (size_t)l * a.kv * max_t;
    const int items = a.n_heads * (HS / kVDims);
    for (int it = blockIdx.x; it < items; it += gridDim.x) {
        const int h = it % a.n_heads, d0 = (it / a.n_heads) * kVDims;
        const float4* kbase = reinterpret_cast<const float4*>(kc + (size_t)(h / kv_mul) * max_t * HS);
        const float* vbase = vc + (size_t)(h / kv_mul) * max_t * HS + d0;
        const float4 qv = reinterpret_cast<const float4*>(a.q + (size_t)h * HS)[min(tid, F4 - 1)];
        // K column f of position t: a uniform base per column plus one 32-bit
        // per-lane offset (the scalar-base load form: no 64-bit address per load)
        const char* kb = reinterpret_cast<const char*>(kbase);
        const size_t kstride = (size_t)max_t * sizeof(float4);
        float4 kr[F4];
        auto load_k = [&](int t, bool skip) {
            if (skip && __builtin_amdgcn_readfirstlane(t) >= n) return;
            const unsigned vo = (unsigned)min(t, n - 1) * (unsigned)sizeof(float4);
#pragma unroll
            for (int f = 0; f < F4; f++) kr[f] = *reinterpret_cast<const float4*>(kb + f * kstride + vo);
        };
        load_k(tid, true);
        float4 vr[kSAVPer];
        auto load_chunk = [&](int c, bool skip) {
#pragma unroll
            for (int k = 0; k < kSAVPer; k++) {
                const int e = tid + kSAThreads * k;
                const int r = e / (kVDims / 4), c4 = e % (kVDims / 4);
                const int t = c * kSAChunk + r;
                if (skip && __builtin_amdgcn_readfirstlane(t) >= n) continue;
                const unsigned vo = ((unsigned)min(t, n - 1) * HS + 4 * c4) * (unsigned)sizeof(float);
                vr[k] = *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(vbase) + vo);
            }
        };
        auto store_chunk = [&](int buf) {
            float* dst = vt + buf * kVDims * kSAStride;
#pragma unroll
            for (int k = 0; k < kSAVPer; k++) {
                const int e = tid + kSAThreads * k;
                const int r = e / (kVDims / 4), c4 = e % (kVDims / 4);
                dst[(4 * c4 + 0) * kSAStride + r] = vr[k].x;
                dst[(4 * c4 + 1) * kSAStride + r] = vr[k].y;
                dst[(4 * c4 + 2) * kSAStride + r] = vr[k].z;
                dst[(4 * c4 + 3) * kSAStride + r] = vr[k].w;
            }
        };
        reinterpret_cast<float4*>(qs)[min(tid, F4 - 1)] = qv;
        wg_bar();   // 1: qs

        float s[kSARounds];
        float m = -INFINITY;
        const float4* q4 = reinterpret_cast<const float4*>(qs);
#pragma unroll
        for (int r = 0; r < kSARounds; r++) {
            s[r] = -INFINITY;
            if (kSAThreads * r >= n) continue;
            const int t = kSAThreads * r + tid;
            if (r > 0) load_k(t, false);
            float score = 0.0f;
#pragma unroll
            for (int f = 0; f < F4; f++) {
                const float4 qf = q4[f];
                score = score + qf.x * kr[f].x;
                score = score + qf.y * kr[f].y;
                score = score + qf.z * kr[f].z;
                score = score + qf.w * kr[f].w;
            }
            if (t < n) {
                s[r] = score / sqrtf((float)HS);
                m = fmaxf(m, s[r]);
            }
        }
        load_chunk(0, true);
        m = group_max<L2Q_WAVE>(m);
        if (lane == 0) red[wv] = m;
        wg_bar();   // 2: wave maxima
        m = red[0];
#pragma unroll
        for (int w = 1; w < kStepCompute; w++) m = fmaxf(m, red[w]);
        float e[kSARounds];
#pragma unroll
        for (int r = 0; r < kSARounds; r++) {
            const int t = kSAThreads * r + tid;
            e[r] = 0.0f;
            if (kSAThreads * r < n && t < n) {
                e[r] = exp_runq_t(s[r] - m, etab);
                p[t] = e[r];
            }
        }
        wg_bar();   // 3: e_t
        if (tid == 0) red[8] = serial_sum(p, n);
        wg_bar();   // 4: sum
        const float sum = red[8];
#pragma unroll
        for (int r = 0; r < kSARounds; r++) {
            const int t = kSAThreads * r + tid;
            if (kSAThreads * r < n && t < n) p[t] = e[r] / sum;
        }
        store_chunk(0);
        wg_bar();   // 5: p_t, first V chunk
        float acc = 0.0f;
        for (int c = 0; c < nchunks; c++) {
            if (c + 1 < nchunks) load_chunk(c + 1, false);
            if (wv == 0 && lane < kVDims) {
                const int tb = c * kSAChunk;
                acc = serial_pv(p + tb, vt + (c & 1) * kVDims * kSAStride + lane * kSAStride, min(kSAChunk, n - tb),
                                acc);
            }
            if (c + 1 < nchunks) store_chunk((c + 1) & 1);
            wg_bar();   // 6..: one per chunk
        }
        st.put(wv == 0 && lane < kVDims, (unsigned)(h * HS + d0 + lane), acc);
    }
}

// ---------------------------------------------------------------------------
// Control wave.

// Workgroup 0 persists the residual stream v of a norm phase (left in LDS
// by the prologue) and, for forward_debug, copies it.
template <int D, int H, int HS>
__device__ __forceinline__ void ctl_persist(const StepArgs& a, int p, const float* L, int lane) {
    using Sh = StepShape<D, H, HS>;
    const int k = phase_kind(p, a.L), l = p / 5;
    float* xout = k == kSQkv ? a.xb : (k == kSW13 ? a.xa : nullptr);
    float* dbg = nullptr;
    if (a.dbg_x && k == kSQkv) dbg = a.dbg_x + (size_t)l * D;
    if (a.dbg_x && k == kSCls) dbg = a.dbg_x + (size_t)a.L * D;
    const float4* in0 = reinterpret_cast<const float4*>(L + Sh::kIn0);
    for (int c = lane; c < D / 4; c += L2Q_WAVE) {
        const float4 v = in0[c];
        if (xout) reinterpret_cast<float4*>(xout)[c] = v;
        if (dbg) reinterpret_cast<float4*>(dbg)[c] = v;
    }
}

// Store the outputs the compute waves staged for phase p.
template <int D, int H, int HS>
__device__ __forceinline__ void ctl_outputs(const StepArgs& a, int p, const float* L, int lane) {
    using Sh = StepShape<D, H, HS>;
    const int k = phase_kind(p, a.L), l = p / 5;
    float* out = k == kSQkv ? a.q : k == kSAtt ? a.att : k == kSWo ? a.wo_out : k == kSW13 ? a.hb
               : k == kSW2 ? a.ffn_out : a.logits;
    float* kc = a.kcache + (size_t)l * a.kv * a.max_t;
    float* vc = a.vcache + (size_t)l * a.kv * a.max_t;
    const unsigned* cnt = reinterpret_cast<const unsigned*>(L + Sh::kCnt);
    const unsigned* off = reinterpret_cast<const unsigned*>(L + Sh::kStOff);
    const float* val = L + Sh::kStVal;
    for (int w = 0; w < kStepCompute; w++) {
        const int n = (int)cnt[w];
        for (int i = lane; i < n; i += L2Q_WAVE) {
            const unsigned o = off[w * kStepStage + i];
            const unsigned e = o & 0x3FFFFFFFu;
            float* base = (o >> 30) == 0 ? out : (o >> 30) == 1 ? kc : vc;
            base[e] = val[w * kStepStage + i];
        }
    }
}

// ---------------------------------------------------------------------------
// The kernel.  Grid = the CU count, every workgroup resident (the host
// checks the occupancy); block = 7 compute waves + the control wave.
template <int D, int H, int HS>
__global__ __launch_bounds__(kStepThreads) void k_step(StepArgs a) {
    using Sh = StepShape<D, H, HS>;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int lane = threadIdx.x & (L2Q_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / L2Q_WAVE);
    const int P = step_phases(a.L);
    float* misc = lds + Sh::kMisc;

    if (wv == kStepCompute) {
        // ---- control wave
        const unsigned epoch = __hip_atomic_load(a.sync.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane < 32) reinterpret_cast<uint64_t*>(misc + 8)[lane] = kExp2Tab[lane];
        if (lane == 0) {
            misc[2] = __int_as_float(a.meta[0]);
            misc[3] = __int_as_float(a.meta[1]);
            misc[1] = 0.0f;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        unsigned kbar = epoch * (unsigned)a.nbar;
        const int n = __float_as_int(misc[3]) + 1;
        const int att_bars = attn_items(a) * (5 + (n + kSAChunk - 1) / kSAChunk);
        for (int p = 0; p < P; p++) {
            const int k = phase_kind(p, a.L);
            bool ok = true;
            STEP_TRACE(p, 0);
            if (p > 0) ok = grid_sync(a.sync, ++kbar, lane);
            STEP_TRACE(p, 1);
            if (lane == 0) misc[1] = ok ? 0.0f : 1.0f;
            STEP_TRACE(p, 2);
            wg_bar();   // B1: barrier passed (or abort)
            if (!ok) return;
            // mirror the compute waves' barriers: a norm phase's prologue (3,
            // v in LDS after the first), a quantize prologue (1), the fold
            // barrier of a GEMV, the attention's
            if (k == kSAtt) {
                for (int i = 0; i < att_bars; i++) wg_bar();
            } else if (k == kSWo || k == kSW2) {
                wg_bar();
                wg_bar();
            } else {
                wg_bar();
                if (blockIdx.x == 0) ctl_persist<D, H, HS>(a, p, lds, lane);
                wg_bar();
                wg_bar();
                wg_bar();
            }
            wg_bar();   // B3: outputs staged
            STEP_TRACE(p, 3);
            ctl_outputs<D, H, HS>(a, p, lds, lane);
        }
        if (blockIdx.x == 0 && lane == 0)
            __hip_atomic_store(a.sync.epoch, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // ---- compute waves
    Slot ring[3];
    Cursor cur;
    cursor_enter<D, H>(a, cur, 0, wv);
    cursor_skip<D, H>(a, cur, wv);
    int next_att = 1;   // phase of the next attention: the ring does not cross it
    issue<D, H>(a, ring[0], cur, next_att, wv, lane);
    issue<D, H>(a, ring[1], cur, next_att, wv, lane);
    issue<D, H>(a, ring[2], cur, next_att, wv, lane);
    int C = 0;
    unsigned* cnt = reinterpret_cast<unsigned*>(lds + Sh::kCnt);
    Stager st{reinterpret_cast<unsigned*>(lds + Sh::kStOff) + wv * kStepStage, lds + Sh::kStVal + wv * kStepStage, 0};
    // one GEMV phase between its barriers B1 (barrier passed) and B3 (outputs
    // staged); false when the control wave has aborted the step
    auto gemv = [&](auto K, int p) {
        wg_bar();   // B1
        if (misc[1] != 0.0f) return false;
        st.n = 0;
        gemv_phase<D, H, HS, K.value>(a, p, ring, C, cur, next_att, lds, wv, lane, st);
        if (lane == 0) cnt[wv] = (unsigned)st.n;
        wg_bar();   // B3
        return true;
    };
    for (int l = 0; l < a.L; l++) {
        if (!gemv(IC<kSQkv>{}, 5 * l)) return;
        wg_bar();   // B1 of the attention
        if (misc[1] != 0.0f) return;
        st.n = 0;
        attn_phase<D, H, HS>(a, l, lds, wv, lane, st);
        if (lane == 0) cnt[wv] = (unsigned)st.n;
        wg_bar();   // B3
        // the attention's loads are done: the held slots go out now
        next_att += 5;
        switch (C % 3) {
            case 0:
                issue<D, H>(a, ring[0], cur, next_att, wv, lane);
                issue<D, H>(a, ring[1], cur, next_att, wv, lane);
                issue<D, H>(a, ring[2], cur, next_att, wv, lane);
                break;
            case 1:
                issue<D, H>(a, ring[1], cur, next_att, wv, lane);
                issue<D, H>(a, ring[2], cur, next_att, wv, lane);
                issue<D, H>(a, ring[0], cur, next_att, wv, lane);
                break;
            default:
                issue<D, H>(a, ring[2], cur, next_att, wv, lane);
                issue<D, H>(a, ring[0], cur, next_att, wv, lane);
                issue<D, H>(a, ring[1], cur, next_att, wv, lane);
                break;
        }
        if (!gemv(IC<kSWo>{}, 5 * l + 2)) return;
        if (!gemv(IC<kSW13>{}, 5 * l + 3)) return;
        if (!gemv(IC<kSW2>{}, 5 * l + 4)) return;
    }
    if (!gemv(IC<kSCls>{}, 5 * a.L)) return;
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
}

}  // namespace l2q
