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

// Activation preparation: xq [T][K] natural order -> xqp [T][K] in the MFMA
// chunk order (INT4: per chunk of G/4 columns, odd columns then even
// columns; INT8: unchanged), sq [T][K/G] = sum of the group's q, xt [T][K/G]
// = q8_bias_term(xs, sq) (runq.c:137).  One thread per (token, group).
template <int BITS, int G>
__global__ __launch_bounds__(256) void k_pf_prep(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                 int K, int T, int8_t* __restrict__ xqp, int* __restrict__ sq,
                                                 float* __restrict__ xt) {
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
    sq[idx] = s;
    xt[idx] = q8_bias_term(xs[idx], s);
}

// Batched GEMM, LDS-staged: workgroup (16*RTW-row tile, 128-token tile),
// 8/TPW waves; wave w computes the RTW 16-row tiles against token tiles
// w, w + 8/TPW, ... (TPW of them; RTW is chosen per shape so that the grid
// covers the CUs).  The columns
// advance in steps of 128 (128/G groups): weights, the permuted activations
// and the step's per-group scalars (xs, xt, sum(q), ws) are loaded with
// coalesced 16-byte loads into registers two steps ahead and written to one
// of two LDS buffers while the other is consumed, one barrier per step.
// Per group: MFMA with the accumulator input 128*sum(q) of the token (x16
// for INT4, whose dot is x16), so D = d + 128*sum(q) (>> 4 for INT4,
// exact), then the ordered fold acc = fma(ws, fma(xs, (float)D, -xt), acc)
// of runq.c:150-156, so every output equals the decode GEMV's bit for bit.
// A step's LDS reads are issued together, then its MFMAs, then the folds in
// group order.
constexpr int kPf2Tokens = 128;
constexpr int kPf2Tpw = 2;                   // token tiles per wave
constexpr int kPf2Threads = 8 / kPf2Tpw * L2Q_WAVE;
constexpr int kPf2Cols = 128;                // columns per LDS step
constexpr int kPf2BPitch = kPf2Cols + 16;    // bytes per token row of the activation stage
template <int BITS>
__host__ __device__ constexpr int pf2_apitch() { return kPf2Cols * BITS / 8 + 16; }
template <int BITS, int G, int RTW>
__host__ __device__ constexpr size_t pf2_stage_bytes() {
    return (size_t)16 * RTW * pf2_apitch<BITS>() + (size_t)kPf2Tokens * kPf2BPitch +
           (size_t)(kPf2Cols / G) * (3 * kPf2Tokens + 16 * RTW) * 4;
}
template <int BITS, int G, int RTW>
__host__ __device__ constexpr size_t pf2_lds_bytes() { return 2 * pf2_stage_bytes<BITS, G, RTW>(); }

template <int BITS, int G, int RTW>
__global__ __launch_bounds__(kPf2Threads) void k_pf_gemm2(
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int rows, int cols,
    const int8_t* __restrict__ xqp, const float* __restrict__ xs, const int* __restrict__ sq,
    const float* __restrict__ xt, int T, float* __restrict__ out, int ldo) {
    constexpr int RT = 16 * RTW;                     // rows per workgroup
    constexpr int KS = kPf2Cols / G;                 // groups per step
    constexpr int AB = kPf2Cols * BITS / 8;          // weight bytes of a row per step
    constexpr int AP = pf2_apitch<BITS>();
    constexpr int GB = G * BITS / 8;                 // weight bytes per group
    constexpr int CB = GB / 4;                       // weight bytes per MFMA lane chunk
    constexpr int CX = G / 4;                        // activation bytes per MFMA lane chunk
    constexpr int AN = RT * AB / 16;                                  // 16-byte weight loads per step
    constexpr int APT = (AN + kPf2Threads - 1) / kPf2Threads;         // per thread
    constexpr int BPT = kPf2Cols * kPf2Tokens / 16 / kPf2Threads;     // 16-byte activation loads per thread
    constexpr int SN = KS * kPf2Tokens;                               // per-token scalars per step
    constexpr int SPT = (SN + kPf2Threads - 1) / kPf2Threads;
    constexpr int WN = KS * RT;                                       // weight scales per step
    constexpr int WPT = (WN + kPf2Threads - 1) / kPf2Threads;
    static_assert(BPT >= 1, "step geometry");
    extern __shared__ __attribute__((aligned(16))) uint8_t pf2_lds[];
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE;
    const int r0 = blockIdx.x * RT, t0 = blockIdx.y * kPf2Tokens;
    const int nb = cols / G, nsteps = (nb + KS - 1) / KS;
    const int rowbytes = cols * BITS / 8;
    const int ntt = min(8, (T - t0 + 15) / 16);      // token tiles of this workgroup
    auto stage = [&](int buf) { return pf2_lds + (size_t)buf * pf2_stage_bytes<BITS, G, RTW>(); };

    // global -> registers for step s (clamped rows / tokens / groups); two
    // register sets, so that step s + 2 is in flight while step s + 1 is
    // written to LDS and step s is consumed.  Every load is unconditional
    // (what lies past a row is zeroed when written to LDS): a load under a
    // condition becomes "zero the register, then a masked load", and the
    // zeroing waits for the loads in flight, which would make the prefetch
    // synchronous.
    struct Regs {
        uint4 ra[APT], rb[BPT];
        float rxs[SPT], rxt[SPT];
        int rsq[SPT];
        float rws[WPT];
    };
    auto fetch = [&](int s, Regs& R) {
#pragma unroll
        for (int k = 0; k < APT; k++) {
            const int e = min(tid + kPf2Threads * k, AN - 1), r = e / (AB / 16), p = e % (AB / 16);
            const int off = min(s * AB + 16 * p, rowbytes - 16);
            R.ra[k] = *reinterpret_cast<const uint4*>(w + (size_t)min(r0 + r, rows - 1) * rowbytes + off);
        }
#pragma unroll
        for (int k = 0; k < BPT; k++) {
            const int e = tid + kPf2Threads * k, t = e / (kPf2Cols / 16), p = e % (kPf2Cols / 16);
            const int off = min(s * kPf2Cols + 16 * p, cols - 16);
            R.rb[k] = *reinterpret_cast<const uint4*>(xqp + (size_t)min(t0 + t, T - 1) * cols + off);
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int e = min(tid + kPf2Threads * k, SN - 1), t = e / KS, g = s * KS + e % KS;
            const size_t gi = (size_t)min(t0 + t, T - 1) * nb + min(g, nb - 1);
            R.rxs[k] = xs[gi];
            R.rxt[k] = xt[gi];
            R.rsq[k] = sq[gi];
        }
#pragma unroll
        for (int k = 0; k < WPT; k++) {
            const int e = min(tid + kPf2Threads * k, WN - 1), r = e / KS, g = s * KS + e % KS;
            R.rws[k] = ws[(size_t)min(r0 + r, rows - 1) * nb + min(g, nb - 1)];
        }
    };
    // registers -> LDS buffer: [A rows][AP] [B tokens][BPitch] [xs][xt][c: KS x 128] [ws: KS x RT]
    auto put = [&](int s, int buf, const Regs& R) {
        uint8_t* A = stage(buf);
        uint8_t* B = A + RT * AP;
        float* S = reinterpret_cast<float*>(B + kPf2Tokens * kPf2BPitch);
#pragma unroll
        for (int k = 0; k < APT; k++) {
            const int e = tid + kPf2Threads * k, r = e / (AB / 16), p = e % (AB / 16);
            const bool in = s * AB + 16 * p < rowbytes;
            if (e < AN) *reinterpret_cast<uint4*>(A + r * AP + 16 * p) = in ? R.ra[k] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < BPT; k++) {
            const int e = tid + kPf2Threads * k, t = e / (kPf2Cols / 16), p = e % (kPf2Cols / 16);
            const bool in = s * kPf2Cols + 16 * p < cols;
            *reinterpret_cast<uint4*>(B + t * kPf2BPitch + 16 * p) = in ? R.rb[k] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int e = tid + kPf2Threads * k, t = e / KS, g = e % KS;
            if (e < SN) {
                S[g * kPf2Tokens + t] = R.rxs[k];
                S[(KS + g) * kPf2Tokens + t] = R.rxt[k];
                reinterpret_cast<int*>(S)[(2 * KS + g) * kPf2Tokens + t] = R.rsq[k] * 128;
            }
        }
#pragma unroll
        for (int k = 0; k < WPT; k++) {
            const int e = tid + kPf2Threads * k;
            if (e < WN) S[3 * KS * kPf2Tokens + (e % KS) * RT + e / KS] = R.rws[k];
        }
    };

    constexpr int TPW = kPf2Tpw, NW = 8 / TPW;
    float acc[TPW][RTW][4];
#pragma unroll
    for (int j = 0; j < TPW; j++)
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[j][i][e] = 0.0f;
    const int c = lane / 16, l16 = lane % 16;
    // token tiles wv + NW*j exist for j < nj (wave-uniform)
    const int nj = wv < ntt ? (ntt - wv + NW - 1) / NW : 0;

    auto compute = [&](int s) {
        if (nj == 0) return;
        const uint8_t* A = stage(s & 1);
        const uint8_t* B = A + RT * AP;
        const float* S = reinterpret_cast<const float*>(B + kPf2Tokens * kPf2BPitch);
        const int ng = min(KS, nb - s * KS);
        // LDS reads of the step: A operands (INT4: x16 nibbles in place), B
        // operand and scalars of every group
        v4i32 av[KS][RTW], bv[KS][TPW];
        long al[KS][RTW], bl[KS][TPW];
        float gxs[KS][TPW], gxt[KS][TPW];
        int cin[KS][TPW];
        float4 wsv[KS][RTW];
#pragma unroll
        for (int g = 0; g < KS; g++) {
            if (g >= ng) break;
#pragma unroll
            for (int i = 0; i < RTW; i++) {
                const uint8_t* pa = A + (16 * i + l16) * AP + g * GB + c * CB;
                if constexpr (G == 64) {
                    if constexpr (BITS == 8) {
                        const int4 v = *reinterpret_cast<const int4*>(pa);
                        av[g][i] = v4i32{v.x, v.y, v.z, v.w};
                    } else {
                        const int2 v = *reinterpret_cast<const int2*>(pa);
                        av[g][i] = v4i32{v.x & (int)0xF0F0F0F0, v.y & (int)0xF0F0F0F0, (v.x << 4) & (int)0xF0F0F0F0,
                                         (v.y << 4) & (int)0xF0F0F0F0};
                    }
                } else {
                    if constexpr (BITS == 8) {
                        const int2 v = *reinterpret_cast<const int2*>(pa);
                        al[g][i] = (long)(unsigned)v.x | ((long)v.y << 32);
                    } else {
                        const int v = *reinterpret_cast<const int*>(pa);
                        al[g][i] = (long)(unsigned)(v & (int)0xF0F0F0F0) | ((long)((v << 4) & (int)0xF0F0F0F0) << 32);
                    }
                }
                wsv[g][i] = *reinterpret_cast<const float4*>(S + 3 * KS * kPf2Tokens + g * RT + 16 * i + 4 * c);
            }
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                const int tl = 16 * (wv + NW * j) + l16;   // token of this lane (in the workgroup)
                const uint8_t* pb = B + tl * kPf2BPitch + g * G + c * CX;
                if constexpr (G == 64) {
                    const int4 v = *reinterpret_cast<const int4*>(pb);
                    bv[g][j] = v4i32{v.x, v.y, v.z, v.w};
                } else {
                    const int2 v = *reinterpret_cast<const int2*>(pb);
                    bl[g][j] = (long)(unsigned)v.x | ((long)v.y << 32);
                }
                gxs[g][j] = S[g * kPf2Tokens + tl];
                gxt[g][j] = S[(KS + g) * kPf2Tokens + tl];
                cin[g][j] = reinterpret_cast<const int*>(S)[(2 * KS + g) * kPf2Tokens + tl];
            }
        }
        // MFMAs of the step
        v4i32 d[KS][TPW][RTW];
#pragma unroll
        for (int g = 0; g < KS; g++) {
            if (g >= ng) break;
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                if (j >= nj) break;
                const v4i32 z4 = {0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < RTW; i++) {
                    if constexpr (G == 64)
                        d[g][j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[g][i], bv[g][j], z4, 0, 0, 0);
                    else
                        d[g][j][i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(al[g][i], bl[g][j], z4, 0, 0, 0);
                }
            }
        }
        // ordered folds
#pragma unroll
        for (int g = 0; g < KS; g++) {
            if (g >= ng) break;
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                if (j >= nj) break;
#pragma unroll
                for (int i = 0; i < RTW; i++) {
                    const float wr[4] = {wsv[g][i].x, wsv[g][i].y, wsv[g][i].z, wsv[g][i].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        // d + 128*sum(q), exact (the INT4 dot is 16x the dot)
                        const int du8 = (BITS == 4 ? d[g][j][i][e] >> 4 : d[g][j][i][e]) + cin[g][j];
                        acc[j][i][e] =
                            __builtin_fmaf(wr[e], __builtin_fmaf(gxs[g][j], (float)du8, -gxt[g][j]), acc[j][i][e]);
                    }
                }
            }
        }
    };
    // step s: fetch s + 2 into the set that held s (written to LDS during
    // step s - 1), consume LDS buffer s & 1, write s + 1 (fetched during
    // step s - 1) to the other buffer.  The fetches are unconditional, past
    // the last step they repeat it: every path then has the same loads in
    // flight, and waiting for one set never waits for the other.
    Regs R0, R1;
    fetch(0, R0);
    fetch(min(1, nsteps - 1), R1);
    put(0, 0, R0);
    __syncthreads();
    for (int s = 0; s < nsteps; s += 2) {
        fetch(min(s + 2, nsteps - 1), R0);
        compute(s);
        if (s + 1 < nsteps) put(s + 1, 1, R1);
        __syncthreads();
        if (s + 1 >= nsteps) break;
        fetch(min(s + 3, nsteps - 1), R1);
        compute(s + 1);
        if (s + 2 < nsteps) put(s + 2, 0, R0);
        __syncthreads();
    }
    // out[t][r]: rows 16i + 4c + e of tile i, token 16 (wv + NW j) + l16
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int t = t0 + 16 * (wv + NW * j) + l16;
        if (j >= nj || t >= T) continue;
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = r0 + 16 * i + 4 * c + e;
                if (r < rows) out[(size_t)t * ldo + r] = acc[j][i][e];
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

// SwiGLU + Q8 quantize of T tokens from interleaved (w1, w3) rows:
// h13 [T][2n] -> xq [T][n], xs [T][n/G], as k_swiglu_quant per token
// (pf.xqp set: also the GEMM operand, pf_emit; xq may then be null).
template <int G>
__global__ __launch_bounds__(256) void k_pf_swiglu_quant(const float* __restrict__ h13, int n, int T,
                                                         int8_t* __restrict__ xq, float* __restrict__ xs,
                                                         PfOperand pf) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   // element of the flattened [T][n]
    const bool in = i < (size_t)T * n;
    float g = 0.0f;
    if (in) {
        const size_t t = i / n, j = i - t * n;
        float h = h13[t * 2 * n + 2 * j];   // (built with -ffp-contract=off, as k_swiglu_quant)
        h *= (1.0f / (1.0f + exp_runq(-h)));
        g = h * h13[t * 2 * n + 2 * j + 1];
    }
    const float s = q8_scale(group_max<G>(fabsf(g)));
    const int q = q8_value_fast(g, s, q8_recip(s));
    if (pf.xqp) pf_emit<G>(pf, i, q, s, in);
    if (in) {
        if (xq) xq[i] = (int8_t)q;
        if ((i % G) == 0) xs[i / G] = s;
    }
}

}  // namespace l2q
