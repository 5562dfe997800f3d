// prefill.h - batched prefill: T tokens through one layer's GEMMs at once.
//
// The decode step streams every weight once per token; a prompt of T tokens
// can share that stream.  Here the group dots of T tokens against a row
// tile come from MFMA (v_mfma_i32_16x16x64_i8 for groups of 64,
// v_mfma_i32_16x16x32_i8 for groups of 32): with K = one group, an MFMA's
// int32 result is exactly the per-(row, token, group) dot, so the fold that
// follows can be the decode path's ordered FMA chain over the groups
// (sum = fma(ws_b, t_b, sum), t_b = fma(xs, (float)(d + 128*sum(q)), -xt),
// runq.c:150-156) and every output is bit-identical to the token-by-token
// forward.  (Batched prefill of the reference: v2-cuda/run.cu:131-162
// matmul_q8_kernel, 347-394 forward_gpu.)
//
// MFMA lane layout (16x16 tiles, checked on gfx950): lane l supplies A row
// l%16 and B column l%16, each with K/4 consecutive-in-K bytes (chunk l/16);
// it receives D rows 4*(l/16)+i, i = 0..3, of column l%16.  A and B share
// the chunk-to-K map, so any permutation of K inside a chunk applied to both
// leaves the dot unchanged: INT4 weights are unpacked in place as 16x their
// odd / even columns (w & 0xF0, (w << 4) & 0xF0, exact) and the activations
// are stored permuted to match, [odd columns | even columns] per chunk.
#pragma once

#include "device.h"
#include "gemv.h"

namespace l2q {

typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// Activation preparation from natural-order xq [T][K], xs [T][K/G]: xqp
// [T][K] in the MFMA chunk order (INT4: per chunk of G/4 columns, odd
// columns then even columns; INT8: unchanged) and the records rec [K/G][T].
// One thread per (token, group).  The producers that quantize write the
// same operand themselves (pf_emit); this serves callers that hold xq.
template <int BITS, int G>
__global__ __launch_bounds__(256) void k_pf_prep(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                 int K, int T, int8_t* __restrict__ xqp, PfRecord* __restrict__ rec) {
    const int nb = K / G;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= T * nb) return;
    const int8_t* src = xq + (size_t)idx * G;   // groups never straddle tokens (K % G == 0)
    int8_t* dst = xqp + (size_t)idx * G;
    int s = 0;
    constexpr int CH = G / 4;                    // columns per MFMA lane chunk
    for (int c = 0; c < 4; c++) {
        for (int j = 0; j < CH; j++) {
            const int8_t v = src[c * CH + j];
            s += v;
            if (BITS == 4) dst[c * CH + (j & 1 ? j / 2 : CH / 2 + j / 2)] = v;
            else dst[c * CH + j] = v;
        }
    }
    const int t = idx / nb, b = idx - t * nb;
    rec[(size_t)b * T + t] = pf_record(xs[idx], s, BITS);
}

// global -> LDS without registers (gfx950 global_load_lds_dword(x4)): lane
// l of the wave writes its SIZE bytes read at src to dst + l * SIZE, dst
// being wave-uniform.  Counted by vmcnt like any load.
template <int SIZE>
__device__ __forceinline__ void dma_lds(const void* src, uint8_t* dst) {
    static_assert(SIZE == 4 || SIZE == 16, "DMA unit");
    if constexpr (SIZE == 16) __builtin_amdgcn_global_load_lds((glb_void_t*)const_cast<void*>(src), (lds_void_t*)dst, 16, 0, 0);
    else __builtin_amdgcn_global_load_lds((glb_void_t*)const_cast<void*>(src), (lds_void_t*)dst, 4, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS bank spreading: the 16-byte units of a row's (a token's) group are
// stored XOR-permuted by a key from the row (token) index, so that the 8
// lanes of a ds_read_b128 phase (16 of a b64 phase), which read the same
// chunk of consecutive rows, fall in distinct banks (32 banks of 4 bytes).
__host__ __device__ constexpr int pf_swz(int units, int x) {
    return units == 4 ? (x >> 1) & 3 : units == 2 ? (x >> 2) & 1 : 0;
}

// Batched GEMM geometry.  A workgroup computes RT rows x TT tokens with
// WR x WT waves, each RTW 16-row tiles x TPW 16-token tiles; the columns
// advance in steps of SC (KS groups).  A step's stage in LDS:
//   A   [KS][RT][GB]   weight bytes of each row and group (GB = G*BITS/8)
//   B   [KS][TT][G]    the tokens' permuted activations
//   R   [KS][TT]       16-byte records (pf_record)
// with the 16-byte units of each row (token) and group permuted by pf_swz
//   W   [KS][RT]       weight scales
// each region filled by 64-lane DMA instructions (16-byte units; 4-byte
// ones for W), instruction k of the stage issued by wave k % NW.
template <int BITS, int G, int RTW, int TPW, int WR, int WT, int SC>
struct Pf3 {
    static constexpr int NW = WR * WT, NT = NW * L2Q_WAVE;
    static constexpr int RT = 16 * RTW * WR, TT = 16 * TPW * WT;
    static constexpr int KS = SC / G;
    static constexpr int GB = G * BITS / 8;
    static constexpr int AU = KS * RT * GB / 16, BU = KS * TT * G / 16, RU = KS * TT, WU = KS * RT;
    static constexpr int NA = (AU + 63) / 64, NB = (BU + 63) / 64, NR = (RU + 63) / 64, NWS = (WU + 63) / 64;
    static constexpr int N = NA + NB + NR + NWS;
    static constexpr int OB = NA * 1024, OR = OB + NB * 1024, OWS = OR + NR * 1024;
    static constexpr int STAGE = OWS + NWS * 256;
    static constexpr int NK = (N + NW - 1) / NW;     // DMA instructions per wave and stage (at most)
    static_assert(SC % G == 0 && SC % 16 == 0 && SC * BITS / 8 >= 16, "step geometry");
};

// Wait for this wave's DMA of every stage but the last K issued: waves
// w < N % NW issue one instruction more per stage.
template <class P, int K>
__device__ __forceinline__ void wait_stages(int wv) {
    if constexpr (P::N % P::NW == 0) {
        wait_vmcnt<K * (P::N / P::NW)>();
    } else {
        if (wv < P::N % P::NW) wait_vmcnt<K * (P::N / P::NW + 1)>();
        else wait_vmcnt<K * (P::N / P::NW)>();
    }
}

// The batched GEMM out[t][r] = sum over groups b, in order, of
// ws[r][b] * fma(xs[t][b], (float)(d + 128*sum(q)), -xt[t][b]), the decode
// GEMV's fold (runq.c:150-156) for every (row, token), bit for bit.  Per
// group: one MFMA per (row tile, token tile) with the record's accumulator
// input, then 3 VALU operations per output (convert, two FMAs; INT4
// weights enter in offset binary, so no shift).  Operands reach LDS by DMA, NST stages in rotation: stage
// s + NST - 1 is requested while stage s is consumed, and one barrier per
// step publishes stage s + 1.  The buffers are distinct LDS variables and
// the loop is unrolled by NST, so the compiler sees which buffer every LDS
// read uses and waits only for DMA into that one.  With PIPE the fold
// trails the MFMAs by one step: step s issues its LDS reads, folds step
// s - 1's MFMA results while they are in flight, then issues its MFMAs,
// whose latency the barrier and the next step's reads cover.  Rows, tokens
// and columns past the ends are clamped into the operands (those outputs
// are never stored).
template <int BITS, int G, int RTW, int TPW, int WR, int WT, int SC, int NST, bool PIPE, int EPI>
__global__ __launch_bounds__(WR * WT * L2Q_WAVE) void k_pf_gemm3(
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int rows, int cols,
    const int8_t* __restrict__ xqp, const PfRecord* __restrict__ rec, int T, float* __restrict__ out, int ldo,
    PfRope rp, PfOperand so) {
    using P = Pf3<BITS, G, RTW, TPW, WR, WT, SC>;
    constexpr int KS = P::KS;
    static_assert(NST >= 3 && NST <= 5, "pipeline depth");
    __shared__ __attribute__((aligned(16))) uint8_t sb0[P::STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sb1[P::STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sb2[P::STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sb3[NST > 3 ? P::STAGE : 16];
    __shared__ __attribute__((aligned(16))) uint8_t sb4[NST > 4 ? P::STAGE : 16];
    uint8_t* const bufs[5] = {sb0, sb1, sb2, sb3, sb4};
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid / L2Q_WAVE);
    const int r0 = blockIdx.x * P::RT, t0 = blockIdx.y * P::TT;
    const int nb = cols / G, nsteps = (cols + SC - 1) / SC, nfull = cols / SC;
    const int rowbytes = cols * BITS / 8;

    // source of this lane's unit in DMA instruction k at step s (clamped;
    // only step 0 is asked for, later steps advance it by `stride`)
    auto src = [&](int k, int s) __attribute__((always_inline)) -> const uint8_t* {
        if (k < P::NA) {
            const int u = min(k * 64 + lane, P::AU - 1);
            const int g = u / (P::RT * P::GB / 16), rem = u % (P::RT * P::GB / 16);
            const int r = rem / (P::GB / 16), part = (rem % (P::GB / 16)) ^ pf_swz(P::GB / 16, r);
            const int col = s * SC + g * G;
            const int off = col < cols ? col * BITS / 8 + part * 16 : rowbytes - 16;
            return w + (size_t)min(r0 + r, rows - 1) * rowbytes + off;
        }
        k -= P::NA;
        if (k < P::NB) {
            const int u = min(k * 64 + lane, P::BU - 1);
            const int g = u / (P::TT * G / 16), rem = u % (P::TT * G / 16);
            const int t = rem / (G / 16), part = (rem % (G / 16)) ^ pf_swz(G / 16, t);
            const int col = s * SC + g * G;
            const int off = col < cols ? col + part * 16 : cols - 16;
            return reinterpret_cast<const uint8_t*>(xqp) + (size_t)min(t0 + t, T - 1) * cols + off;
        }
        k -= P::NB;
        if (k < P::NR) {
            const int u = min(k * 64 + lane, P::RU - 1);
            const int g = u / P::TT, t = u % P::TT;
            return reinterpret_cast<const uint8_t*>(rec + (size_t)min(s * KS + g, nb - 1) * T + min(t0 + t, T - 1));
        }
        k -= P::NR;
        const int u = min(k * 64 + lane, P::WU - 1);
        const int g = u / P::RT, r = u % P::RT;
        return reinterpret_cast<const uint8_t*>(ws + (size_t)min(r0 + r, rows - 1) * nb + min(s * KS + g, nb - 1));
    };
    // bytes one instruction's sources advance per full step
    auto stride = [&](int k) __attribute__((always_inline)) -> size_t {
        if (k < P::NA) return (size_t)SC * BITS / 8;
        if (k < P::NA + P::NB) return (size_t)SC;
        if (k < P::NA + P::NB + P::NR) return (size_t)KS * T * sizeof(PfRecord);
        return (size_t)KS * 4;
    };
    const uint8_t* p0[P::NK];
#pragma unroll
    for (int kk = 0; kk < P::NK; kk++) p0[kk] = src(min(wv + P::NW * kk, P::N - 1), 0);
    // step s: every unit's source is its step-0 source advanced s steps; in
    // a last, partial step the units of groups past the end (whose sources
    // would lie past the rows) are masked off: unit u of a region with UG
    // units per group belongs to group u / UG, so a lane of instruction k
    // (the region's k-th) is live when lane < ng * UG - 64 * k (wave-uniform
    // bound)
    auto issue = [&](int s, uint8_t* buf) __attribute__((always_inline)) {
        const bool full = s < nfull;
        const int ng = min(KS, nb - s * KS);
#pragma unroll
        for (int kk = 0; kk < P::NK; kk++) {
            const int k = wv + P::NW * kk;
            if (k < P::N) {
                const uint8_t* a = p0[kk] + (size_t)s * stride(k);
                if (k < P::NA) {
                    if (full || lane < ng * (P::RT * P::GB / 16) - 64 * k) dma_lds<16>(a, buf + k * 1024);
                } else if (k < P::NA + P::NB) {
                    const int kb = k - P::NA;
                    if (full || lane < ng * (P::TT * G / 16) - 64 * kb) dma_lds<16>(a, buf + P::OB + kb * 1024);
                } else if (k < P::NA + P::NB + P::NR) {
                    const int kr = k - P::NA - P::NB;
                    if (full || lane < ng * P::TT - 64 * kr) dma_lds<16>(a, buf + P::OR + kr * 1024);
                } else {
                    const int kw = k - P::NA - P::NB - P::NR;
                    if (full || lane < ng * P::RT - 64 * kw) dma_lds<4>(a, buf + P::OWS + kw * 256);
                }
            }
        }
    };

    constexpr int CB = P::GB / 4, CX = G / 4;    // bytes per MFMA lane chunk: weights, activations
    const int c = lane / 16, l16 = lane % 16;
    // this lane's chunk within its row's / token's group after pf_swz (rows
    // and tokens of a lane differ by multiples of 16, which leave the key)
    const int offa = 16 * ((c * CB / 16) ^ pf_swz(P::GB / 16, l16)) + c * CB % 16;
    const int offb = 16 * ((c * CX / 16) ^ pf_swz(G / 16, l16)) + c * CX % 16;
    const int rw0 = (wv % WR) * 16 * RTW, tw0 = (wv / WR) * 16 * TPW;
    const int left = T - t0 - tw0;
    const int nj = left <= 0 ? 0 : min(TPW, (left + 15) / 16);   // token tiles with tokens (wave-uniform)
    float acc[TPW][RTW][4];
#pragma unroll
    for (int j = 0; j < TPW; j++)
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[j][i][e] = 0.0f;

    // a step's operands read from LDS, and what its fold needs
    struct Ops {
        v4i32 av[KS][RTW], bv[KS][TPW], cin[KS][TPW];
        long al[KS][RTW], bl[KS][TPW];
    };
    struct Pend {
        v4i32 d[KS][TPW][RTW];
        float2 sc[KS][TPW];      // xs, xt
        float4 wsv[KS][RTW];
        int ng;
    };
    auto read = [&](int s, const uint8_t* buf, Ops& o, Pend& pn) __attribute__((always_inline)) {
        pn.ng = min(KS, nb - s * KS);
#pragma unroll
        for (int g = 0; g < KS; g++) {
#pragma unroll
            for (int i = 0; i < RTW; i++) {
                const uint8_t* pa = buf + (g * P::RT + rw0 + 16 * i + l16) * P::GB + offa;
                if constexpr (G == 64) {
                    if constexpr (BITS == 8) {
                        const int4 v = *reinterpret_cast<const int4*>(pa);
                        o.av[g][i] = v4i32{v.x, v.y, v.z, v.w};
                    } else {
                        const int2 v = *reinterpret_cast<const int2*>(pa);
                        o.av[g][i] = v4i32{v.x, v.y, 0, 0};
                    }
                } else {
                    if constexpr (BITS == 8) {
                        const int2 v = *reinterpret_cast<const int2*>(pa);
                        o.al[g][i] = (long)(unsigned)v.x | ((long)v.y << 32);
                    } else {
                        o.al[g][i] = (long)(unsigned)*reinterpret_cast<const int*>(pa);
                    }
                }
                pn.wsv[g][i] = *reinterpret_cast<const float4*>(buf + P::OWS + (g * P::RT + rw0 + 16 * i + 4 * c) * 4);
            }
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                const int tl = tw0 + 16 * j + l16;
                const uint8_t* pb = buf + P::OB + (g * P::TT + tl) * G + offb;
                if constexpr (G == 64) {
                    const int4 v = *reinterpret_cast<const int4*>(pb);
                    o.bv[g][j] = v4i32{v.x, v.y, v.z, v.w};
                } else {
                    const int2 v = *reinterpret_cast<const int2*>(pb);
                    o.bl[g][j] = (long)(unsigned)v.x | ((long)v.y << 32);
                }
                // the record (c, xs, xt): c is the accumulator input of every row
                const int4 ci = *reinterpret_cast<const int4*>(buf + P::OR + (g * P::TT + tl) * 16);
                o.cin[g][j] = v4i32{ci.x, ci.x, ci.x, ci.x};
                pn.sc[g][j] = make_float2(__int_as_float(ci.y), __int_as_float(ci.z));
            }
        }
    };
    auto mfma = [&](Ops& o, Pend& pn) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < KS; g++) {
            if (g < pn.ng) {
                // INT4: the odd / even nibbles as bytes in offset binary (n ^ 8 =
                // s4(n) + 8, 0..15), matching the activations' [odd | even] order
                // per chunk; the record's c adds the remaining 120*sum(q)
                if constexpr (BITS == 4) {
                    constexpr int kLo = 0x0F0F0F0F, kFlip = (int)0x88888888;
#pragma unroll
                    for (int i = 0; i < RTW; i++) {
                        if constexpr (G == 64) {
                            const int x = o.av[g][i][0] ^ kFlip, y = o.av[g][i][1] ^ kFlip;
                            o.av[g][i] = v4i32{(int)((unsigned)x >> 4) & kLo, (int)((unsigned)y >> 4) & kLo, x & kLo,
                                               y & kLo};
                        } else {
                            const int v = (int)o.al[g][i] ^ kFlip;
                            o.al[g][i] = (long)(unsigned)((int)((unsigned)v >> 4) & kLo) | ((long)(v & kLo) << 32);
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    if (j < nj) {
#pragma unroll
                        for (int i = 0; i < RTW; i++) {
                            if constexpr (G == 64)
                                pn.d[g][j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.av[g][i], o.bv[g][j], o.cin[g][j], 0, 0, 0);
                            else
                                pn.d[g][j][i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(o.al[g][i], o.bl[g][j], o.cin[g][j], 0, 0, 0);
                        }
                    }
                }
            }
        }
    };
    auto fold = [&](const Pend& pn) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < KS; g++) {
            if (g < pn.ng) {
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    if (j < nj) {
#pragma unroll
                        for (int i = 0; i < RTW; i++) {
                            const float wr[4] = {pn.wsv[g][i].x, pn.wsv[g][i].y, pn.wsv[g][i].z, pn.wsv[g][i].w};
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                const int dv = pn.d[g][j][i][e];
                                acc[j][i][e] = __builtin_fmaf(
                                    wr[e], __builtin_fmaf(pn.sc[g][j].x, (float)dv, -pn.sc[g][j].y),
                                    acc[j][i][e]);
                            }
                        }
                    }
                }
            }
        }
    };
    auto barrier = []() __attribute__((always_inline)) { asm volatile("s_barrier" ::: "memory"); };
    // step s (buffer k = s % NST): request stage s + NST - 1; read stage s;
    // fold step s - 1; MFMAs of step s; wait for this wave's part of stage
    // s + 1; barrier (every wave's part of s + 1 has landed and every wave
    // is done reading stage s, which the next step refills)
    Pend pa, pb;       // MFMA results of even / odd steps
    pa.ng = pb.ng = 0;
    auto step = [&](int s, int k, Pend& cur, Pend& prev) __attribute__((always_inline)) {
        if (s + NST - 1 < nsteps) issue(s + NST - 1, bufs[(k + NST - 1) % NST]);
        Ops o;
        if (nj > 0) read(s, bufs[k], o, cur);
        if constexpr (PIPE) {
            if (nj > 0 && s > 0) fold(prev);
            if (nj > 0) mfma(o, cur);
        } else if (nj > 0) {
            mfma(o, cur);
            fold(cur);
        }
        if (s + 1 < nsteps) {
            if (s + NST - 1 < nsteps) wait_stages<P, NST - 2>(wv);
            else wait_vmcnt<0>();
            barrier();
        }
    };
#pragma unroll
    for (int i = 0; i < NST - 1; i++)
        if (i < nsteps) issue(i, bufs[i]);
    if (nsteps >= NST - 1) wait_stages<P, NST - 2>(wv);
    else wait_vmcnt<0>();
    barrier();
    // unrolled by 2 * NST: buffer and result set both known at compile time
    for (int s = 0; s < nsteps; s += 2 * NST) {
#pragma unroll
        for (int k = 0; k < 2 * NST; k++)
            if (s + k < nsteps) {
                if (k % 2 == 0) step(s + k, k % NST, pa, pb);
                else step(s + k, k % NST, pb, pa);
            }
    }
    if (PIPE && nj > 0) fold((nsteps - 1) % 2 == 0 ? pa : pb);
    if constexpr (EPI == 2) {
        // SwiGLU + Q8 into the w2 GEMM's operand (so): rows alternate w1 / w3
        // of a hidden unit, the workgroup's RT = 2G rows are one quantization
        // group of G units; g = (h1 * (1/(1+expf(-h1)))) * h3 (runq.c:
        // 405-410, the operations of k_swiglu_quant), its group's max over
        // the lanes of the token (xor 16 / 32) and the WR row-waves (LDS),
        // Q8 as k_swiglu_quant quantizes (runq.c:117-139)
        static_assert(TPW == 1 && P::RT == 2 * G, "one token tile per wave, one group per workgroup");
        static_assert(2 * WT * WR * 16 * sizeof(float) <= P::STAGE, "the exchange fits in stage buffer 0");
        const int t = t0 + tw0 + l16;
        const bool tin = nj > 0 && t < T;
        float gv[RTW][2];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                float h = acc[0][i][2 * m];
                h *= (1.0f / (1.0f + exp_runq(-h)));
                gv[i][m] = tin ? h * acc[0][i][2 * m + 1] : 0.0f;
                amax = fmaxf(amax, fabsf(gv[i][m]));
            }
        unsigned ua, ub;
        xor16_pair(__float_as_uint(amax), ua, ub);
        amax = fmaxf(__uint_as_float(ua), __uint_as_float(ub));
        xor32_pair(__float_as_uint(amax), ua, ub);
        amax = fmaxf(__uint_as_float(ua), __uint_as_float(ub));
        const int wr = wv % WR, wt = wv / WR;
        float* xm = reinterpret_cast<float*>(sb0);      // [WT][WR][16] row-wave maxima
        int* xq = reinterpret_cast<int*>(xm + WT * WR * 16);   // [WT][WR][16] row-wave sums
        // __syncthreads, not the loop's bare s_barrier: these LDS stores must
        // land (lgkmcnt(0)) before other waves read them
        __syncthreads();   // every wave is past its last LDS read of the stages
        if (c == 0) xm[(wt * WR + wr) * 16 + l16] = amax;
        __syncthreads();
        float gm = 0.0f;
#pragma unroll
        for (int k = 0; k < WR; k++) gm = fmaxf(gm, xm[(wt * WR + k) * 16 + l16]);
        const float s = q8_scale(gm);
        const float r = q8_recip(s);
        int qv[RTW][2];
        int qs = 0;
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                qv[i][m] = q8_value_fast(gv[i][m], s, r);
                qs += qv[i][m];
            }
        xor16_pair((unsigned)qs, ua, ub);
        qs = (int)(ua + ub);
        xor32_pair((unsigned)qs, ua, ub);
        qs = (int)(ua + ub);
        if (c == 0) xq[(wt * WR + wr) * 16 + l16] = qs;
        __syncthreads();
        if (!tin) return;
        int total = 0;
#pragma unroll
        for (int k = 0; k < WR; k++) total += xq[(wt * WR + k) * 16 + l16];
        constexpr int CH = G / 4;
        int8_t* dst = so.xqp + (size_t)t * so.K + r0 / 2;   // the group's G bytes of token t
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const int j = 16 * RTW * wr / 2 + 8 * i + 2 * c + m;   // unit of the group
                const int jj = j % CH;
                dst[so.bits == 4 ? j - jj + ((jj & 1) ? jj / 2 : CH / 2 + jj / 2) : j] = (int8_t)qv[i][m];
            }
        if (wr == 0 && c == 0) so.rec[(size_t)(r0 / P::RT) * T + t] = pf_record(s, total, so.bits);
        return;
    }
    // out[t][r]: rows 16i + 4c + e of the wave's tile i, token 16j + l16
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int t = t0 + tw0 + 16 * j + l16;
        if (j >= nj || t >= T) continue;
#pragma unroll
        for (int i = 0; i < RTW; i++) {
            const int r = r0 + rw0 + 16 * i + 4 * c;
            float* o = out + (size_t)t * ldo + r;
            if constexpr (EPI == 1) {
                // pairs (r, r + 1), (r + 2, r + 3): r is a multiple of 4
                const int pos = rp.pos0 + t, crow = rp.row0 + t;
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    const int rr = r + 2 * m;
                    if (rr >= rows) continue;
                    const float v0 = acc[j][i][2 * m], v1 = acc[j][i][2 * m + 1];
                    if (rr < rp.dim + rp.kv_dim) {
                        const int e = rr < rp.dim ? rr : rr - rp.dim;
                        const int hd = e % rp.hs;
                        const float cs = rp.rope[(size_t)pos * rp.hs + hd];
                        const float sn = rp.rope[(size_t)pos * rp.hs + hd + 1];
                        const float a0 = __builtin_fmaf(v0, cs, -(v1 * sn));
                        const float a1 = __builtin_fmaf(v0, sn, v1 * cs);
                        if (rr < rp.dim) {
                            o[2 * m] = a0;
                            o[2 * m + 1] = a1;
                        } else {
                            const size_t ko = k_index(rp.k_il, e / rp.hs, crow, hd, rp.hs, rp.max_t);
                            rp.kcache[ko] = a0;
                            rp.kcache[ko + 1] = a1;
                        }
                    } else {
                        const int e = rr - rp.dim - rp.kv_dim;
                        const size_t vo = ((size_t)(e / rp.hs) * rp.max_t + crow) * rp.hs + e % rp.hs;
                        rp.vcache[vo] = v0;
                        rp.vcache[vo + 1] = v1;
                    }
                }
                continue;
            }
            if (r + 3 < rows && (ldo & 3) == 0 && (reinterpret_cast<uintptr_t>(o) & 15) == 0) {
                *reinterpret_cast<float4*>(o) = make_float4(acc[j][i][0], acc[j][i][1], acc[j][i][2], acc[j][i][3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (r + e < rows) o[e] = acc[j][i][e];
            }
        }
    }
}

// Residual add + RMSNorm + Q8 of T vectors into the GEMM operand
// (runq.c:294-305 then :117-139), with the operations of the decode GEMV's
// kNorm prologue (prologue_compute): v = x + resid, the sum of squares in
// the reference's order (runq_sumsq_t over a transposed LDS copy), inv =
// 1/sqrtf(ss/n + 1e-5), o = w * (inv * v), group maxima of |o| on the bit
// patterns, q8 values.  Workgroup (split s, token t) of 256 threads, thread
// i holding float4 chunks c = i + 256k: every split forms the token's whole
// sum of squares (the chain is latency, not work), and quantizes, stores
// and emits the chunks with k % kPfNormSplit == s, so a token's
// quantization is spread over kPfNormSplit CUs.  A group is G/4
// consecutive lanes.  xout receives v.
constexpr int kPfNormThreads = 256, kPfNormSplit = 2, kPfNormMaxChunks = 8;   // n <= 8192
template <int G>
__global__ __launch_bounds__(kPfNormThreads) void k_pf_rmsnorm_quant(
    const float* __restrict__ x, const float* __restrict__ resid, float* __restrict__ xout,
    const float* __restrict__ w, int n, PfOperand pf) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float vt[16 * sumsq_stride(kPfNormThreads * kPfNormMaxChunks * 4)];
    __shared__ float inv_s;
    const int tid = threadIdx.x, sp = blockIdx.x, t = blockIdx.y;
    const int nc = n / 4, st = sumsq_stride(n);
    const size_t to = (size_t)t * n;
    const float4* x4 = reinterpret_cast<const float4*>(x + to);
    const float4* r4 = resid ? reinterpret_cast<const float4*>(resid + to) : nullptr;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[kPfNormMaxChunks], rv[kPfNormMaxChunks], wv[kPfNormMaxChunks];
    // every load first: one round trip
#pragma unroll
    for (int k = 0; k < kPfNormMaxChunks; k++) {
        const int c = tid + kPfNormThreads * k;
        if (c < nc) {
            v[k] = x4[c];
            if (resid) rv[k] = r4[c];
            if (k % kPfNormSplit == sp) wv[k] = w4[c];
        }
    }
#pragma unroll
    for (int k = 0; k < kPfNormMaxChunks; k++) {
        const int c = tid + kPfNormThreads * k;
        if (c < nc) {
            if (resid) { v[k].x += rv[k].x; v[k].y += rv[k].y; v[k].z += rv[k].z; v[k].w += rv[k].w; }
            const int e = 4 * c;   // elements e..e+3: accumulators e%16.., step e/16
            vt[((e + 0) & 15) * st + (e >> 4)] = v[k].x;
            vt[((e + 1) & 15) * st + (e >> 4)] = v[k].y;
            vt[((e + 2) & 15) * st + (e >> 4)] = v[k].z;
            vt[((e + 3) & 15) * st + (e >> 4)] = v[k].w;
            if (xout && k % kPfNormSplit == sp) reinterpret_cast<float4*>(xout + to)[c] = v[k];
        }
    }
    __syncthreads();
    if (tid < L2Q_WAVE) {
        const float ss = runq_sumsq_t(vt, n, st, tid);
        if (tid == 0) inv_s = 1.0f / sqrtf(ss / (float)n + 1e-5f);
    }
    __syncthreads();
    const float inv = inv_s;
    constexpr int CH = G / 4;   // the INT4 operand's permutation unit (pf_emit)
#pragma unroll
    for (int k = 0; k < kPfNormMaxChunks; k++) {
        if (kPfNormThreads * k >= nc) break;   // uniform across the workgroup
        if (k % kPfNormSplit != sp) continue;
        const int c = tid + kPfNormThreads * k;
        const bool in = c < nc;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (in) {
            o.x = wv[k].x * (inv * v[k].x); o.y = wv[k].y * (inv * v[k].y);
            o.z = wv[k].z * (inv * v[k].z); o.w = wv[k].w * (inv * v[k].w);
        }
        unsigned mb = max(max(__float_as_uint(o.x) & 0x7fffffffu, __float_as_uint(o.y) & 0x7fffffffu),
                          max(__float_as_uint(o.z) & 0x7fffffffu, __float_as_uint(o.w) & 0x7fffffffu));
        mb = group_umax<G / 4>(mb);
        const float sc = q8_scale(__uint_as_float(mb));
        const float r = q8_recip(sc);
        const int q0 = q8_value_fast(o.x, sc, r), q1 = q8_value_fast(o.y, sc, r);
        const int q2 = q8_value_fast(o.z, sc, r), q3 = q8_value_fast(o.w, sc, r);
        const int sum = group_isum<G / 4>(in ? q0 + q1 + q2 + q3 : 0);   // exact in any order
        if (in) {
            const int e = 4 * c;
            int8_t* row = pf.xqp + (size_t)t * pf.K;
            auto b2 = [](int a, int b) __attribute__((always_inline)) {
                return (uint16_t)((a & 0xff) | ((b & 0xff) << 8));
            };
            if (pf.bits == 4) {   // chunk of CH: odd elements first, then even (pf_emit's order)
                const int cb = e - e % CH, m = (e % CH) / 4;
                *reinterpret_cast<uint16_t*>(row + cb + 2 * m) = b2(q1, q3);
                *reinterpret_cast<uint16_t*>(row + cb + CH / 2 + 2 * m) = b2(q0, q2);
            } else {
                *reinterpret_cast<unsigned*>(row + e) = (unsigned)b2(q0, q1) | ((unsigned)b2(q2, q3) << 16);
            }
            if (c % (G / 4) == 0) pf.rec[(size_t)(e / G) * pf.T + t] = pf_record(sc, sum, pf.bits);
        }
    }
}

// Gather the embedding rows of T tokens: x[t] = emb[tokens[t]].
__global__ void k_pf_embed(const float* __restrict__ emb, const int* __restrict__ tokens, float* __restrict__ x,
                           int dim) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < dim) x[(size_t)t * dim + i] = emb[(size_t)tokens[t] * dim + i];
}

}  // namespace l2q
