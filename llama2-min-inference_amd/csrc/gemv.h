// gemv.h - batch-1 GEMV over group-quantized INT8 / packed-INT4 weights,
// with the prologues and epilogues of the decode step fused in.
//
// out[r] = sum_b ws[r,b] * (xs[b] * d_u8(r,b) - xt[b])  (runq.c:142-159)
// with d(r,b) = sum_{j<G} w[r,bG+j] * xq[bG+j] the exact int32 group dot,
// d_u8 = d + 128*sum(xq_b) and xt[b] = xs[b]*128*sum(xq_b).
//
// Mapping (wave64, no MFMA: at batch 1 this is a pure weight stream):
//   - rows are cut into units of PR consecutive rows, dealt round-robin:
//     wave w of W takes units w, w + W, w + 2W, ..., so every wave has the
//     same number (+-1) and the grid sweeps the matrix front to back, all
//     waves reading one window of ~W units at a time (better DRAM locality
//     than a contiguous range per wave: measured 2-3% faster on every shape);
//   - a row is read in sweeps of 1 KiB: in sweep s lane j loads the 16
//     bytes at s*1024 + 16*j, so every load instruction of a wave covers
//     one contiguous KiB (the best-coalesced form of the stream); the
//     row's group scales are loaded by all 64 lanes (one dword each);
//   - the next unit's loads are issued while the current unit is consumed
//     (a ring of PR rows in registers), so loads are always in flight;
//   - a group spans P = G*BITS/128 consecutive lanes (1, 2 or 4); their
//     partial int32 dots and activation sums are combined with DPP lane
//     moves, exactly (integer adds);
//   - the activation chunk a lane needs is the same for every row, so it is
//     loaded (or taken from the prologue's LDS copy) once into registers;
//   - INT4 nibbles are consumed in place (see dot8_q4_x16): no unpack to
//     bytes, two v_dot4_i32_i8 per 8 weights;
//   - per-(row, group) terms and scales go to LDS and one lane per row
//     folds them in group order, sum = fma(ws_b, t_b, sum), reproducing the
//     reference's float accumulation bit for bit; the PR rows of a unit are
//     folded by PR lanes at once, with the LDS reads issued ahead.
//
// Prologues (how the activation vector reaches the lanes):
//   kPreq   int8 activations + scales already in HBM (xq, xs);
//   kQuant  fp32 vector x_in (cols), Q8-quantized by each workgroup into LDS
//           (runq.c:117-139; the attention output before wo, the SwiGLU
//           output before w2);
//   kNorm   residual add v = x_in + resid (x_in = emb[token] when emb is
//           set), RMSNorm in the reference's exact order, Q8 quantize, into
//           LDS (runq.c:294-305 + :117-139); workgroup 0 also stores v to
//           x_out (the persisted residual stream).  Every workgroup computes
//           the same bits, so no grid-wide step is needed.
// Epilogues:
//   kStore  out[r] = sum;
//   kRopeKV rows [0,dim) are q, [dim,dim+kv) k, [dim+kv,dim+2kv) v of a
//           layer: q and k are rotated with the host-built (cos, sin) table
//           (runq.c:351-365) and k, v appended to the cache at meta[1];
//   kSwiglu rows alternate w1/w3 of one hidden unit: out[h] =
//           (h1 * (1/(1+expf(-h1)))) * h3 (runq.c:405-410).
#pragma once
#include "device.h"
#include "exp_runq.h"

namespace l2q {

enum GemvPro { kPreq = 0, kQuant = 1, kNorm = 2 };
enum GemvEpi { kStore = 0, kRopeKV = 1, kSwiglu = 2 };

struct GemvArgs {
    float* out;
    const int8_t* xq;        // kPreq
    const float* xs;         // kPreq
    const void* w;
    const float* ws;
    int rows;
    int cols;
    int32_t* dots;           // optional [rows][cols/G] int32 group dots
    // prologue
    const float* x_in;       // kQuant / kNorm
    const float* emb;        // kNorm: x_in = emb + meta[0]*cols when set
    const float* resid;      // kNorm, optional
    float* x_out;            // kNorm, optional (written by workgroup 0)
    const float* norm_w;     // kNorm
    const int* meta;         // {token, pos}
    // epilogue (kRopeKV)
    int dim, kv_dim, hs, max_t;
    float* kcache;
    float* vcache;
    const float* rope;
    int kv_stage;            // 1: k/v rows written at position 0 (a staging row, max_t 1)
    int k_il;                // K cache layout (see k_index)
};


constexpr int kSweepBytes = 16 * L2Q_WAVE;   // one 128-bit load per lane
// Rows per unit (PR): (even, odd) pairs for the pair epilogues; single rows
// for plain stores of long rows (>= 5 sweeps), whose two-row unit would
// crowd the registers and leave a wave one unit with nothing to overlap.
__host__ __device__ constexpr int gemv_unit_rows(int NS, int EPI) { return EPI == 0 && NS >= 5 ? 1 : 2; }

__host__ __device__ constexpr int gemv_sweeps(int bits, int cols) { return (cols * bits / 8 + kSweepBytes - 1) / kSweepBytes; }

// One workgroup of 8 waves (2 per SIMD) per CU: the workgroup-wide prologue
// is then shared by every wave of the CU instead of being recomputed by
// several workgroups.  (12 waves for short rows measured ~1% slower in the
// decode step: a 4096-row matrix then fills only 171 of the 256 CUs.)  Rows
// of two sweeps may run 11 waves where that fills the grid's last round of
// units better (see go_gemv).
__host__ __device__ constexpr int gemv_waves(int) { return 8; }
constexpr int kGemvWavesWide = 11;

// Rows folded at once per wave (F lanes run F ordered FMA chains side by
// side): the fold's instructions are issued for the whole wave whatever the
// number of active lanes, so batching rows divides their cost by F/PR.  F
// is 8, or 4 / 2 where the fold area would exceed 96 KiB of LDS.
constexpr size_t kGemvFoldBudget = 96 * 1024;
__host__ __device__ constexpr int gemv_nbp(int nb);
__host__ __device__ constexpr int gemv_fold_rows(int nb, int waves) {
    return (size_t)waves * 2 * 8 * gemv_nbp(nb) * 4 <= kGemvFoldBudget   ? 8
           : (size_t)waves * 2 * 4 * gemv_nbp(nb) * 4 <= kGemvFoldBudget ? 4
                                                                          : 2;
}

// Scale sweeps (64 dwords each) for rows of at most NS weight sweeps.
__host__ __device__ constexpr int gemv_scale_sweeps(int bits, int group, int NS) {
    return (NS * kSweepBytes * 8 / bits / group + L2Q_WAVE - 1) / L2Q_WAVE;
}

// A prologue thread holds ceil(cols/4/threads) float4 chunks of the input;
// with cols*BITS/8 <= 1024*NS that is at most ceil(NS*2048/(BITS*threads)).
__host__ __device__ constexpr int prologue_chunks(int NS, int BITS, int threads) {
    return (NS * 2048 / BITS + threads - 1) / threads;
}

// Row stride (floats) of the per-wave fold area: nb rounded up to a float4,
// plus one float4 so that the PR folding lanes start on different banks.
__host__ __device__ constexpr int gemv_nbp(int nb) { return (nb + 3) / 4 * 4 + 4; }

// Row stride (floats) of the transposed norm input: row l holds elements
// l, l+16, l+32, ... (one reference FMA accumulator each), padded to a
// float4 multiple plus one float4 so that 16 lanes reading float4s at the
// same step hit distinct banks.
__host__ __device__ constexpr int sumsq_stride(int n) { return ((n + 15) / 16 + 3) / 4 * 4 + 4; }

// LDS layout: [fold: waves x (terms, scales) x F x nbp floats]
//             [act_q: cols int8, padded to 32 B][act_s: nb floats, padded to 4]
//             [vt: the residual sum, transposed for the norm chains (kNorm): 16 x sumsq_stride(cols) floats]
//             [misc: 4 floats | exp table: 32 doubles]
constexpr int kGemvMiscFloats = 4 + 64;
// RoPE values held per lane by the kRopeKV epilogue (head size <= 256)
constexpr int kRopeRegs = kAttnMaxHs / L2Q_WAVE;
__host__ __device__ constexpr size_t gemv_fold_floats(int nb, int waves) {
    return (size_t)waves * 2 * gemv_fold_rows(nb, waves) * gemv_nbp(nb);
}
//
// Rows of more than 4 sweeps keep the activations in LDS (read per chunk)
// instead of registers, which keeps the kernel at two or more waves per
// SIMD; the INT4 form is stored pre-split per 32-element chunk as
// [even-column dwords E0..E3 | odd-column dwords O0..O3] (see act_split_addr).
__host__ __device__ constexpr bool gemv_act_lds(int NS) { return NS > 4; }
__host__ __device__ constexpr size_t gemv_lds_bytes(int pro, int cols, int group, int bits, int PR,
                                                    int waves = gemv_waves(0)) {
    return gemv_fold_floats(cols / group, waves) * sizeof(float) +
           (pro == kPreq && !gemv_act_lds(gemv_sweeps(bits, cols))
                ? 0
                : (size_t)(cols + 31) / 32 * 32 + (size_t)(cols / group + 3) / 4 * 16) +
           (pro == kNorm ? (size_t)16 * sumsq_stride(cols) * sizeof(float) : 0) + kGemvMiscFloats * sizeof(float);
}

// Byte address of element e in the pre-split INT4 activation layout.
__device__ __forceinline__ int act_split_addr(int e) {
    return (e & ~31) + ((e & 1) << 4) + (((e >> 3) & 3) << 2) + ((e & 7) >> 1);
}

// Geometry of one 16-byte lane chunk.
template <int BITS, int G>
struct Chunk {
    static constexpr int EL = 16 * 8 / BITS;        // elements per chunk (32 INT4, 16 INT8)
    static constexpr int AD = EL / 4;               // activation dwords per chunk (= 32 / BITS)
    static constexpr int GB = G * BITS / 8;         // weight bytes per group
    static constexpr int P = GB / 16;               // lanes per group
    static_assert(GB % 16 == 0 && kSweepBytes % GB == 0, "unsupported group");
};

// Activation chunks of a lane, held in registers for all rows (x only when
// the activations are not read from LDS).
template <int BITS, int G, int NS, bool XR = true>
struct LaneActs {
    int x[XR ? NS : 1][32 / BITS];   // INT8: natural order; INT4: [even dwords | odd dwords] per 8 elements
    float xs[NS];                    // scale of the chunk's group
    float xt[NS];                    // bias term of the group (runq.c:137)
    int sq[NS];                      // sum(q) over the whole group
};

// Raw activation words of lane chunk (s, lane): loads only.  Every load is
// issued (lanes past the row read the last chunk and zero it afterwards),
// so the number of loads in flight is known to the compiler and waiting
// for these never waits for the weight loads issued after them.
template <int BITS, int G, int NS>
__device__ __forceinline__ void load_lane_raw(int (&raw)[NS][32 / BITS], float (&sc)[NS], const int8_t* xq,
                                              const float* xs, int cols, int lane) {
    using C = Chunk<BITS, G>;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int e0 = (s * kSweepBytes + 16 * lane) * 8 / BITS;   // first element of the chunk
        const int ec = min(e0, cols - C::EL);
        const uint4* p = reinterpret_cast<const uint4*>(xq + ec);
#pragma unroll
        for (int v = 0; v < C::AD / 4; v++) {
            const uint4 u = p[v];
            raw[s][4 * v + 0] = (int)u.x; raw[s][4 * v + 1] = (int)u.y;
            raw[s][4 * v + 2] = (int)u.z; raw[s][4 * v + 3] = (int)u.w;
        }
        sc[s] = xs[ec / G];
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
        if ((s * kSweepBytes + 16 * lane) * 8 / BITS >= cols) {
#pragma unroll
            for (int k = 0; k < C::AD; k++) raw[s][k] = 0;
            sc[s] = 0.0f;
        }
    }
}

// Sum over the P lanes of a group (P = 1, 2, 4): exact integer adds.
template <int P>
__device__ __forceinline__ int group_lanes_isum(int v) {
    return group_isum<P>(v);
}

// sum(q) over the group, the bias term and (INT4) the even/odd byte split.
template <int BITS, int G, int NS>
__device__ __forceinline__ void finish_lane_acts(LaneActs<BITS, G, NS, true>& A, const int (&raw)[NS][32 / BITS],
                                                 const float (&sc)[NS]) {
    using C = Chunk<BITS, G>;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        int q = 0;
#pragma unroll
        for (int k = 0; k < C::AD; k++) q = dot4(raw[s][k], 0x01010101, q);
        q = group_lanes_isum<C::P>(q);
        A.sq[s] = q;
        A.xs[s] = sc[s];
        A.xt[s] = q8_bias_term(sc[s], q);
        if (BITS == 4) {
#pragma unroll
            for (int k = 0; k < C::AD / 2; k++) {
                A.x[s][k] = even_bytes(raw[s][2 * k], raw[s][2 * k + 1]);
                A.x[s][C::AD / 2 + k] = odd_bytes(raw[s][2 * k], raw[s][2 * k + 1]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < C::AD; k++) A.x[s][k] = raw[s][k];
        }
    }
}

// Partial int32 dot of one 16-byte weight chunk against the lane's
// activation dwords x (x16 for INT4).
template <int BITS>
__device__ __forceinline__ int chunk_dot_x(const uint4 w, const int* x) {
    if (BITS == 8) {
        int d = dot4((int)w.x, x[0], 0);
        d = dot4((int)w.y, x[1], d);
        d = dot4((int)w.z, x[2], d);
        return dot4((int)w.w, x[3], d);
    } else {
        int d = dot8_q4_x16(w.x, x[0], x[4], 0);
        d = dot8_q4_x16(w.y, x[1], x[5], d);
        d = dot8_q4_x16(w.z, x[2], x[6], d);
        return dot8_q4_x16(w.w, x[3], x[7], d);
    }
}

template <int BITS, int G, int NS>
__device__ __forceinline__ int chunk_dot(const uint4 w, const LaneActs<BITS, G, NS, true>& A, int s) {
    return chunk_dot_x<BITS>(w, A.x[s]);
}

// The lane's activation dwords of the chunk starting at element e0, from
// the LDS copy (INT8 natural order, INT4 pre-split): 16 or 32 bytes.
template <int BITS>
__device__ __forceinline__ void lds_chunk(const int8_t* act, int e0, int (&x)[32 / BITS]) {
    const int4* p = reinterpret_cast<const int4*>(act + e0);
    const int4 v = p[0];
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    if (BITS == 4) {
        const int4 u = p[1];
        x[4] = u.x; x[5] = u.y; x[6] = u.z; x[7] = u.w;
    }
}

// Per-sweep scale, bias term and group sum of q for a lane whose
// activations stay in LDS.
template <int BITS, int G, int NS>
__device__ __forceinline__ void lane_scalars_lds(LaneActs<BITS, G, NS, false>& A, const int8_t* act,
                                                 const float* act_s, int cols, int lane) {
    using C = Chunk<BITS, G>;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int e0 = (s * kSweepBytes + 16 * lane) * 8 / BITS;
        int q = 0;
        float sc = 0.0f;
        if (e0 < cols) {
            int x[32 / BITS];
            lds_chunk<BITS>(act, e0, x);
#pragma unroll
            for (int k = 0; k < C::AD; k++) q = dot4(x[k], 0x01010101, q);
            sc = act_s[e0 / G];
        }
        q = group_lanes_isum<C::P>(q);
        A.sq[s] = q;
        A.xs[s] = sc;
        A.xt[s] = q8_bias_term(sc, q);
    }
}

// Sum of squares of v[0..n) in the reference's order (runq.c:295-302):
// lanes 0..15 of the calling wave each run one of its 16 FMA accumulators
// (j = l, l+16, ...), then the _mm512_reduce_add_ps tree, then the tail as
// GCC compiles the scalar loop (a block of 8 unfused, then FMAs).  The
// result is valid in lane 0.  v is in LDS; all 64 lanes must call.  The
// next block's 16 reads are issued before the current block's FMAs, so
// the chain waits on LDS only once.
__device__ __forceinline__ float runq_sumsq(const float* v, int n, int lane) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (lane < 16) {
        const int nfull = n & ~15;
        const int nblk = nfull / 256;
        float a[16], b[16];
        auto rd = [&](float (&dst)[16], int blk) {
            const int j = (blk < nblk ? blk : nblk - 1) * 256;
#pragma unroll
            for (int u = 0; u < 16; u++) dst[u] = v[j + 16 * u + lane];
        };
        auto chain = [&](const float (&src)[16]) {
#pragma unroll
            for (int u = 0; u < 16; u++) acc = __builtin_fmaf(src[u], src[u], acc);
        };
        if (nblk > 0) {
            rd(a, 0);
            for (int blk = 0; blk < nblk; blk += 2) {
                rd(b, blk + 1);                     // in flight during a's chain
                __builtin_amdgcn_sched_barrier(0);
                chain(a);
                __builtin_amdgcn_sched_barrier(0);
                if (blk + 1 >= nblk) break;
                rd(a, blk + 2);
                __builtin_amdgcn_sched_barrier(0);
                chain(b);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        for (int j = nblk * 256; j < nfull; j += 16) {
            const float e = v[j + lane];
            acc = __builtin_fmaf(e, e, acc);
        }
    }
    acc = __shfl_down(acc, 8, 16) + acc;
    acc = __shfl_down(acc, 4, 16) + acc;
    const float p = acc + __shfl_down(acc, 2, 16);
    float s = p + __shfl_down(p, 1, 16);
    if (lane == 0) {
        int j = n & ~15;
        if (n - j >= 8)
            for (int e = 0; e < 8; e++, j++) s = s + v[j] * v[j];
        for (; j < n; j++) s = __builtin_fmaf(v[j], v[j], s);
    }
    return s;
}

// runq_sumsq over the transposed copy vt (row l = accumulator l's elements
// in order, see sumsq_stride): the same operations in the same order, each
// lane reading its own chain with float4 loads issued a block ahead.
__device__ __forceinline__ float runq_sumsq_t(const float* vt, int n, int stride, int lane) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (lane < 16) {
        const int steps = (n & ~15) / 16;             // chain length
        const float4* p = reinterpret_cast<const float4*>(vt + lane * stride);
        const int nblk = steps / 32;                  // blocks of 8 float4
        float4 a[8], b[8];
        auto rd = [&](float4 (&d)[8], int blk) {
            const int q = (blk < nblk ? blk : nblk - 1) * 8;
#pragma unroll
            for (int u = 0; u < 8; u++) d[u] = p[q + u];
        };
        auto chain = [&](const float4 (&v)[8]) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                acc = __builtin_fmaf(v[u].x, v[u].x, acc);
                acc = __builtin_fmaf(v[u].y, v[u].y, acc);
                acc = __builtin_fmaf(v[u].z, v[u].z, acc);
                acc = __builtin_fmaf(v[u].w, v[u].w, acc);
            }
        };
        if (nblk > 0) {
            rd(a, 0);
            for (int blk = 0; blk < nblk; blk += 2) {
                rd(b, blk + 1);
                chain(a);
                if (blk + 1 >= nblk) break;
                rd(a, blk + 2);
                chain(b);
            }
        }
        for (int k = nblk * 32; k < steps; k++) acc = __builtin_fmaf(vt[lane * stride + k], vt[lane * stride + k], acc);
    }
    acc = __shfl_down(acc, 8, 16) + acc;
    acc = __shfl_down(acc, 4, 16) + acc;
    const float p = acc + __shfl_down(acc, 2, 16);
    float s = p + __shfl_down(p, 1, 16);
    if (lane == 0) {
        int j = n & ~15;
        auto at = [&](int e) { return vt[(e & 15) * stride + (e >> 4)]; };
        if (n - j >= 8)
            for (int e = 0; e < 8; e++, j++) s = s + at(j) * at(j);
        for (; j < n; j++) s = __builtin_fmaf(at(j), at(j), s);
    }
    return s;
}

// Workgroup prologue: quantize (for kNorm: residual add + RMSNorm first) the
// fp32 vector into LDS act_q[cols] / act_s[nb].  Thread t handles float4
// chunks c = t + 256*k (elements 4c..4c+3); a group is G/4 consecutive
// threads of one wave, so group maxima are DPP lane-group reductions.  The
// inputs were loaded to registers by the caller before the weight loads.
template <int G, int PRO, int PC, int RC, bool SPLIT, int THREADS>
__device__ __forceinline__ void prologue_compute(const GemvArgs& a, float4 (&xin)[PC], const float4 (&res)[RC],
                                                 const float4 (&nw)[RC], int8_t* act_q, float* act_s, float* vs,
                                                 float* misc, int nchunks) {
#pragma clang fp contract(off)
    constexpr int kProChunks = PC;
    const int tid = threadIdx.x;
    const int lane = tid & (L2Q_WAVE - 1);
    const int n = a.cols;
    float inv = 1.0f;
    if constexpr (PRO == kNorm) {
#pragma unroll
        for (int k = 0; k < kProChunks; k++) {
            const int c = tid + THREADS * k;
            if (c < nchunks) {
                float4 v = xin[k];
                if (a.resid) { v.x += res[k].x; v.y += res[k].y; v.z += res[k].z; v.w += res[k].w; }
                xin[k] = v;
                const int st = sumsq_stride(n);
                const int e = 4 * c;   // elements e..e+3: accumulators e%16.., step e/16
                vs[((e + 0) & 15) * st + (e >> 4)] = v.x;
                vs[((e + 1) & 15) * st + (e >> 4)] = v.y;
                vs[((e + 2) & 15) * st + (e >> 4)] = v.z;
                vs[((e + 3) & 15) * st + (e >> 4)] = v.w;
                if (a.x_out && blockIdx.x == 0) *reinterpret_cast<float4*>(a.x_out + 4 * c) = v;
            }
        }
        __syncthreads();
        if (tid < L2Q_WAVE) {
            const float ss = runq_sumsq_t(vs, n, sumsq_stride(n), lane);
            if (lane == 0) misc[0] = 1.0f / sqrtf(ss / (float)n + 1e-5f);
        }
        __syncthreads();
        inv = misc[0];
    }
#pragma unroll
    for (int k = 0; k < kProChunks; k++) {
        if (THREADS * k >= nchunks) break;   // uniform across the workgroup
        const int c = tid + THREADS * k;
        const bool in = c < nchunks;
        float4 o = xin[k];
        if constexpr (PRO == kNorm) {
            o.x = nw[k].x * (inv * o.x); o.y = nw[k].y * (inv * o.y);
            o.z = nw[k].z * (inv * o.z); o.w = nw[k].w * (inv * o.w);
        }
        if (!in) o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        // the group maximum of |o| on the bit patterns (a NaN would win here
        // where fmaxf drops it; the reference quantizer has no defined result
        // for one either)
        unsigned mb = max(max(__float_as_uint(o.x) & 0x7fffffffu, __float_as_uint(o.y) & 0x7fffffffu),
                          max(__float_as_uint(o.z) & 0x7fffffffu, __float_as_uint(o.w) & 0x7fffffffu));
        mb = group_umax<G / 4>(mb);
        const float s = q8_scale(__uint_as_float(mb));
        const float r = q8_recip(s);
        if (in) {
            // int8 values in the low bytes (q8_byte_fast), packed by byte permutes
            const unsigned b0 = q8_byte_fast(o.x, s, r), b1 = q8_byte_fast(o.y, s, r);
            const unsigned b2 = q8_byte_fast(o.z, s, r), b3 = q8_byte_fast(o.w, s, r);
            constexpr unsigned kLoBytes = 0x0c0c0400u;   // byte 0 of lo, byte 0 of hi, zeros
            if (SPLIT) {   // INT4 pre-split layout: (q0, q2) to E, (q1, q3) to O
                *reinterpret_cast<uint16_t*>(act_q + act_split_addr(4 * c)) = (uint16_t)__builtin_amdgcn_perm(b2, b0, kLoBytes);
                *reinterpret_cast<uint16_t*>(act_q + act_split_addr(4 * c + 1)) = (uint16_t)__builtin_amdgcn_perm(b3, b1, kLoBytes);
            } else {
                const unsigned lo = __builtin_amdgcn_perm(b1, b0, kLoBytes), hi = __builtin_amdgcn_perm(b3, b2, kLoBytes);
                reinterpret_cast<unsigned*>(act_q)[c] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
            }
            if ((c % (G / 4)) == 0) act_s[c / (G / 4)] = s;
        }
    }
    __syncthreads();
}

// Ordered fold of one row: sum_b fma(ws_b, t_b, sum) for b = 0..nb-1.  The
// terms and scales stream from LDS through a ring of R blocks of 4 groups,
// each block loaded R-1 blocks ahead of the FMA chain, so the chain never
// waits on LDS and no registers are copied between iterations.  Loads run
// up to R blocks past the row (into the next row's area, or the activation
// area after the last one: always inside the workgroup's LDS); what they
// read is never folded.
template <int R = 6>
__device__ __forceinline__ float fold_row(const float* tp, const float* sp, int nb) {
    const float4* t4 = reinterpret_cast<const float4*>(tp);
    const float4* s4 = reinterpret_cast<const float4*>(sp);
    const int nfull = nb >> 2;             // whole blocks of 4 groups
    const int rem = nb & 3;                // groups in a trailing partial block
    float4 T[R], S[R];
#pragma unroll
    for (int j = 0; j < R; j++) {
        T[j] = t4[j];
        S[j] = s4[j];
    }
    float sum = 0.0f;
    int b = 0;
    for (; b + R <= nfull; b += R) {
#pragma unroll
        for (int j = 0; j < R; j++) {
            sum = __builtin_fmaf(S[j].x, T[j].x, sum);
            sum = __builtin_fmaf(S[j].y, T[j].y, sum);
            sum = __builtin_fmaf(S[j].z, T[j].z, sum);
            sum = __builtin_fmaf(S[j].w, T[j].w, sum);
            // keep the reload after the block's last use, so the slot's
            // registers are reused rather than copied
            __builtin_amdgcn_sched_barrier(0);
            T[j] = t4[b + j + R];
            S[j] = s4[b + j + R];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // slot j now holds block b + j: fewer than R whole blocks remain, then
    // possibly one partial block
#pragma unroll
    for (int j = 0; j < R; j++) {
        if (b + j < nfull) {
            sum = __builtin_fmaf(S[j].x, T[j].x, sum);
            sum = __builtin_fmaf(S[j].y, T[j].y, sum);
            sum = __builtin_fmaf(S[j].z, T[j].z, sum);
            sum = __builtin_fmaf(S[j].w, T[j].w, sum);
        } else if (b + j == nfull && rem) {
            sum = __builtin_fmaf(S[j].x, T[j].x, sum);
            if (rem > 1) sum = __builtin_fmaf(S[j].y, T[j].y, sum);
            if (rem > 2) sum = __builtin_fmaf(S[j].z, T[j].z, sum);
        }
    }
    return sum;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Persistent over units of PR rows: local unit j of wave w is the grid's
// unit w + j*W (U units, W waves, j < ceil((U - w)/W)); fold batches and
// the loop count local units.  The wave's first unit is loaded
// before the prologue (which runs once per workgroup while it streams in);
// unit u+1 is loaded as soon as unit u has been consumed.  Terms of F rows
// (F/PR units) are collected before one ordered fold on F lanes.  A wave
// without units loads row 0 (never used), so every path issues the same
// loads and no wait covers younger loads than it must.
template <int BITS, int G, int NS, int PRO, int EPI, int PR, int W>
__global__ __launch_bounds__(W * L2Q_WAVE) void k_gemv(GemvArgs a) {
    constexpr int WAVES = W;
    constexpr int THREADS = WAVES * L2Q_WAVE;
    static_assert(PR == gemv_unit_rows(NS, EPI), "unit size");
    using C = Chunk<BITS, G>;
    constexpr int NSS = gemv_scale_sweeps(BITS, G, NS);
    constexpr bool ACTL = gemv_act_lds(NS);           // activations read from LDS per chunk
    constexpr bool SPLIT = ACTL && BITS == 4;
    static_assert(PR % 2 == 0 || EPI == kStore, "pair epilogues need an even unit");
    static_assert(EPI == kStore || PRO == kNorm, "fused epilogues run after the norm prologue");
    // Read every kernel argument into SGPRs here, before any of them is used:
    // the scalar loads then share one round trip to the argument buffer
    // instead of costing one each at their first uses.
    asm volatile("" ::"s"(a.rows), "s"(a.cols), "s"(a.w), "s"(a.ws), "s"(a.x_in), "s"(a.emb), "s"(a.resid),
                 "s"(a.norm_w), "s"(a.xq), "s"(a.xs), "s"(a.meta), "s"(a.out), "s"(gridDim.x));
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int lane = threadIdx.x & (L2Q_WAVE - 1);
    const int wv = threadIdx.x / L2Q_WAVE;
    const int nb = a.cols / G;
    const int nbp = gemv_nbp(nb);
    const int F = gemv_fold_rows(nb, WAVES);   // rows per fold batch
    const int UB = F / PR;                     // units per fold batch (1, 2, 4 or 8)
    const int ubm = UB - 1;                    // x % UB == x & ubm
    float* tb = lds + (size_t)wv * 2 * F * nbp;
    float* sb = tb + F * nbp;
    int8_t* act_q = reinterpret_cast<int8_t*>(lds + gemv_fold_floats(nb, WAVES));
    float* act_s = reinterpret_cast<float*>(act_q + (a.cols + 31) / 32 * 32);
    float* vs = act_s + (nb + 3) / 4 * 4;
    float* misc = vs + (PRO == kNorm ? 16 * sumsq_stride(a.cols) : 0);
    uint64_t* etab = reinterpret_cast<uint64_t*>(misc + 4);   // exp table (kSwiglu)
    const int rowbytes = a.cols * BITS / 8;
    const uint8_t* wbase = static_cast<const uint8_t*>(a.w);
    const bool leader = (lane % C::P) == 0;

    const int nunits = (a.rows + PR - 1) / PR;
    const int nwaves = gridDim.x * WAVES;
    const int gw = blockIdx.x * WAVES + wv;
    // units dealt round-robin: local unit j of this wave is gw + j*nwaves
    const int u0 = 0;
    const int u1 = gw < nunits ? (nunits - gw + nwaves - 1) / nwaves : 0;

    // 1. prologue inputs first, so that waiting for them never waits on the
    //    weight loads issued after them (vector loads complete in order)
    constexpr int kProChunks = PRO == kPreq ? 1 : prologue_chunks(NS, BITS, THREADS);
    constexpr int kResChunks = PRO == kNorm ? kProChunks : 1;
    float4 xin[kProChunks], res[kResChunks], nw[kResChunks];
    const int nchunks = a.cols / 4;
    if (PRO != kPreq) {
        // unconditional loads (clamped chunk index; see load_lane_raw)
        // meta (written by the host each step) is read only for the embedding
        // row of the first layer: a scalar load from memory the other loads
        // would otherwise wait behind
        const float* src = a.x_in;
        if (PRO == kNorm && a.emb) src = a.emb + (size_t)__builtin_nontemporal_load(a.meta) * a.cols;
        const float* rsrc = (PRO == kNorm && a.resid) ? a.resid : src;
#pragma unroll
        for (int k = 0; k < kProChunks; k++) {
            const int c = min((int)threadIdx.x + THREADS * k, nchunks - 1);
            xin[k] = reinterpret_cast<const float4*>(src)[c];
            if constexpr (PRO == kNorm) {
                res[k] = reinterpret_cast<const float4*>(rsrc)[c];
                nw[k] = reinterpret_cast<const float4*>(a.norm_w)[c];
            }
        }
    }
    // epilogue tables: loaded with the prologue inputs, stored to LDS by the
    // prologue, so the epilogue never waits on a global load queued behind
    // the weight stream
    uint64_t etab_v = 0;
    if (EPI == kSwiglu) etab_v = kExp2Tab[threadIdx.x & 31];
    // the position, for the RoPE row: loaded ahead of the weights, so that
    // addressing the row waits for nothing behind it
    int pos = 0;
    if (EPI == kRopeKV) pos = a.meta[1];
    int raw[ACTL ? 1 : NS][32 / BITS];
    float sc[ACTL ? 1 : NS];
    constexpr int kCopyChunks = ACTL && PRO == kPreq ? (NS * 512 / BITS + THREADS - 1) / THREADS : 1;   // 16-byte xq chunks
    constexpr int kXsChunks = ACTL && PRO == kPreq ? (NS * kSweepBytes * 8 / BITS / G + THREADS - 1) / THREADS : 1;
    uint4 xcp[kCopyChunks];
    float xsv[kXsChunks];
    const int ncopy = a.cols / 16;
    if (PRO == kPreq) {
        if constexpr (!ACTL) {
            load_lane_raw<BITS, G, NS>(raw, sc, a.xq, a.xs, a.cols, lane);
        } else {
#pragma unroll
            for (int k = 0; k < kCopyChunks; k++)
                xcp[k] = reinterpret_cast<const uint4*>(a.xq)[min((int)threadIdx.x + THREADS * k, ncopy - 1)];
#pragma unroll
            for (int k = 0; k < kXsChunks; k++) xsv[k] = a.xs[min((int)threadIdx.x + THREADS * k, nb - 1)];
        }
    }
#if L2Q_INPUT_FIRST
    // a computing prologue: let its inputs arrive before this grid's weight
    // requests queue in front of them (measured: faster in the decode step;
    // pre-quantized inputs are better left to arrive with the weights).  A
    // grid of one unit per wave has nothing to overlap with its only weight
    // load, which then goes out first (uniform branch).
    if (PRO != kPreq && nunits > nwaves) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
#endif
    __builtin_amdgcn_sched_barrier(0);

    // 2. weight loads: every load is issued unconditionally (addresses past
    //    the row are clamped to valid ones, units past the wave's range read
    //    row 0; neither value is used), so the in-flight count is the same on
    //    every path and waits never cover more than they must
    uint4 w4[PR][NS];
    float wsv[PR][NSS];
    auto load_unit = [&](int u) {
        const bool real = u < u1;
#pragma unroll
        for (int k = 0; k < PR; k++) {
            const int row = real ? min((gw + u * nwaves) * PR + k, a.rows - 1) : 0;
            const uint8_t* p = wbase + (size_t)row * rowbytes;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                int off = s * kSweepBytes + 16 * lane;
                if (s == NS - 1) off = min(off, rowbytes - 16);
                w4[k][s] = load_stream(p + off);
            }
            const float* q = a.ws + (size_t)row * nb;
#pragma unroll
            for (int ss = 0; ss < NSS; ss++) wsv[k][ss] = q[min(ss * L2Q_WAVE + lane, nb - 1)];
        }
    };
    const bool has_work = u0 < u1;   // wave-uniform
    load_unit(u0);
    __builtin_amdgcn_sched_barrier(0);
    // the RoPE row of this position: its address needs meta, so it is
    // issued after everything that does not
    // the RoPE row of the position, kRopeRegs values per lane (element
    // lane + 64k in register k), gathered by the fold's epilogue
    float rope_r[kRopeRegs] = {};
    if (EPI == kRopeKV) {
#pragma unroll
        for (int k = 0; k < kRopeRegs; k++) rope_r[k] = a.rope[(size_t)pos * a.hs + min(lane + 64 * k, a.hs - 1)];
    }

    // 3. prologue (workgroup-wide) while the weights stream in
    // every thread stores its entry (duplicates write the same value): a
    // store under a thread condition lets the compiler sink the table load
    // behind the weight loads, where waiting for it waits for them
    if (EPI == kSwiglu) etab[threadIdx.x & 31] = etab_v;
    if (PRO != kPreq) {
        prologue_compute<G, PRO, kProChunks, kResChunks, SPLIT, THREADS>(a, xin, res, nw, act_q, act_s, vs, misc, nchunks);
        if constexpr (!ACTL) load_lane_raw<BITS, G, NS>(raw, sc, act_q, act_s, a.cols, lane);
    } else if constexpr (ACTL) {
        // copy xq (and xs) into LDS, INT4 in the pre-split layout
#pragma unroll
        for (int k = 0; k < kCopyChunks; k++) {
            const int c = threadIdx.x + THREADS * k;
            if (c < ncopy) {
                const uint4 v = xcp[k];
                if (SPLIT) {
                    const int e0 = 16 * c;
                    uint2 ev, od;
                    ev.x = (unsigned)even_bytes((int)v.x, (int)v.y); ev.y = (unsigned)even_bytes((int)v.z, (int)v.w);
                    od.x = (unsigned)odd_bytes((int)v.x, (int)v.y); od.y = (unsigned)odd_bytes((int)v.z, (int)v.w);
                    *reinterpret_cast<uint2*>(act_q + act_split_addr(e0)) = ev;
                    *reinterpret_cast<uint2*>(act_q + act_split_addr(e0 + 1)) = od;
                } else {
                    reinterpret_cast<uint4*>(act_q)[c] = v;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kXsChunks; k++) {
            const int i = threadIdx.x + THREADS * k;
            if (i < nb) act_s[i] = xsv[k];
        }
        __syncthreads();
    }
    if (!has_work) return;
    LaneActs<BITS, G, NS, !ACTL> A;
    if constexpr (ACTL) lane_scalars_lds<BITS, G, NS>(A, act_q, act_s, a.cols, lane);
    else finish_lane_acts<BITS, G, NS>(A, raw, sc);

    // dots and per-group terms of row k of unit u into fold-batch row br
    auto consume_row = [&](int k, int u) {
        const int row = (gw + u * nwaves) * PR + k;
        const int br = ((u - u0) & ubm) * PR + k;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int off = s * kSweepBytes + 16 * lane;
            int dp;
            if constexpr (ACTL) {
                // lanes past the row read a valid chunk; their dots are never used
                int x[32 / BITS];
                lds_chunk<BITS>(act_q, min(off * 8 / BITS, a.cols - C::EL), x);
                dp = chunk_dot_x<BITS>(w4[k][s], x);
            } else {
                dp = chunk_dot<BITS, G, NS>(w4[k][s], A, s);
            }
            int d = group_lanes_isum<C::P>(dp);
            if (BITS == 4) d >>= 4;   // exact: the x16 dot is a multiple of 16
            if (leader && off < rowbytes) {
                const int g = off / C::GB;
                if (a.dots && row < a.rows) a.dots[(size_t)row * nb + g] = d;
                tb[br * nbp + g] = group_term(A.xs[s], A.xt[s], d, A.sq[s]);
            }
        }
#pragma unroll
        for (int ss = 0; ss < NSS; ss++) {
            const int g = ss * L2Q_WAVE + lane;
            if (g < nb) sb[br * nbp + g] = wsv[k][ss];
        }
    };

    // ordered fold of a batch of nrows rows (local units from j0 on) on
    // lanes 0..nrows-1, then the epilogue
    auto fold_batch = [&](int j0, int nrows) {
        wave_lds_sync();
        float sum = 0.0f;
        if (lane < nrows) sum = fold_row(tb + lane * nbp, sb + lane * nbp, nb);
        const bool mine = lane < nrows;
        const int row = (gw + (j0 + lane / PR) * nwaves) * PR + lane % PR;
        if (EPI == kStore) {
            if (mine && row < a.rows) a.out[row] = sum;
        } else if (EPI == kRopeKV) {
            // rows come in (even, odd) pairs held by lanes (0,1), (2,3), ...
            const float other = dpp_f<kDppXor1>(sum);
            // x / hs without an integer division: for 0 <= x < 2^24 and
            // hs <= 256, umulhi(x, floor((2^32-1)/hs) + 1) is the exact
            // quotient (the multiplier exceeds 2^32/hs by less than 1, so
            // the error x*(m - 2^32/hs)/2^32 stays below 1/hs)
            const unsigned hs_m = 0xFFFFFFFFu / (unsigned)a.hs + 1u;
            auto hsdiv = [&](int x) { return (int)__umulhi((unsigned)x, hs_m); };
            // (cos, sin) of this lane's pair, gathered from the RoPE
            // registers by every lane (a permute reads any lane's value)
            const int e = row < a.dim ? row : row - a.dim;
            const int eg = hsdiv(e);                      // head of the row
            const int hd = (e & ~1) - eg * a.hs;          // even element of the pair (hs is even)
            float c = 0.0f, s = 0.0f;
#pragma unroll
            for (int k = 0; k < kRopeRegs; k++) {
                const float ck = __shfl(rope_r[k], hd & 63);
                const float sk = __shfl(rope_r[k], (hd + 1) & 63);
                if ((hd >> 6) == k) { c = ck; s = sk; }
            }
            const int cpos = a.kv_stage ? 0 : pos;
            if (mine && row < a.rows) {
                const bool odd = row & 1;
                const float v0 = odd ? other : sum, v1 = odd ? sum : other;
                if (row < a.dim + a.kv_dim) {            // q or k: rotate
                    const float r = odd ? __builtin_fmaf(v0, s, v1 * c) : __builtin_fmaf(v0, c, -(v1 * s));
                    if (row < a.dim) a.out[row] = r;
                    else a.kcache[k_index(a.k_il, eg, cpos, e - eg * a.hs, a.hs, a.max_t)] = r;
                } else {                                  // v: appended as is
                    const int ev = row - a.dim - a.kv_dim;
                    const int gv = hsdiv(ev);
                    a.vcache[((size_t)gv * a.max_t + cpos) * a.hs + (ev - gv * a.hs)] = sum;
                }
            }
        } else {   // kSwiglu: (w1, w3) pairs on lanes (0,1), (2,3), ...
            const float h3 = dpp_f<kDppXor1>(sum);
            if (mine && (lane & 1) == 0 && row < a.rows) {
#pragma clang fp contract(off)
                float h = sum;
                h *= (1.0f / (1.0f + exp_runq_t(-h, etab)));
                a.out[row >> 1] = h * h3;
            }
        }
        // the fold area is reused by the next unit: keep its term writes
        // behind this unit's fold reads
        wave_lds_sync();
    };

    for (int u = u0; u + 1 < u1; u++) {
#pragma unroll
        for (int k = 0; k < PR; k++) consume_row(k, u);
        // the unit's registers are free again: the next unit streams in
        __builtin_amdgcn_sched_barrier(0);
        load_unit(u + 1);
        __builtin_amdgcn_sched_barrier(0);
        if (((u - u0 + 1) & ubm) == 0) fold_batch(u + 1 - UB, F);
    }
#pragma unroll
    for (int k = 0; k < PR; k++) consume_row(k, u1 - 1);
    const int last = ((u1 - u0 - 1) & ubm) + 1;   // units in the last batch
    fold_batch(u1 - last, last * PR);
}

}  // namespace l2q
