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

constexpr int kPfTile = 16;          // rows and tokens per MFMA tile
constexpr int kPfWaves = 4;          // waves per workgroup

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

// A operand: row r's chunk of group b (K/4 columns) as int8, 16x for INT4.
template <int BITS, int G>
__device__ __forceinline__ void pf_load_a(const uint8_t* wrow, int b, int kq, int (&a)[G / 16]) {
    constexpr int CH = G / 4;                    // columns in this lane's chunk
    if (BITS == 8) {
        const int* p = reinterpret_cast<const int*>(wrow + (size_t)b * G + kq * CH);
#pragma unroll
        for (int i = 0; i < CH / 4; i++) a[i] = p[i];
    } else {
        // CH columns = CH/2 bytes: odd columns (high nibbles) then even ones
        const int* p = reinterpret_cast<const int*>(wrow + ((size_t)b * G + kq * CH) / 2);
#pragma unroll
        for (int i = 0; i < CH / 8; i++) {
            const int w = p[i];
            a[i] = w & (int)0xF0F0F0F0;
            a[CH / 8 + i] = (w << 4) & (int)0xF0F0F0F0;
        }
    }
}

// Batched GEMM with the exact ordered fold: out[t][r] for t < T, r < rows.
// Wave (row tile, token group of NT token tiles): the weight tile of a
// group is loaded once for NT MFMAs; the operands of group b+1 are loaded
// while group b is folded (two register sets, the loop unrolled by two so
// neither set is copied).  Waves of one row tile are adjacent, so they share
// the weight tile through L2.
template <int BITS, int G, int NT>
struct PfOperands {
    int a[G / 16];
    int bx[NT][G / 16];
    float ws4[4];
    float gxs[NT], gxt[NT];
    int gsq[NT];
};

template <int BITS, int G, int NT>
__global__ __launch_bounds__(kPfWaves * L2Q_WAVE) void k_pf_gemm(
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int rows, int cols,
    const int8_t* __restrict__ xqp, const float* __restrict__ xs, const int* __restrict__ sq,
    const float* __restrict__ xt, int T, float* __restrict__ out, int ldo) {
    const int lane = threadIdx.x & (L2Q_WAVE - 1);
    const int gw = blockIdx.x * kPfWaves + threadIdx.x / L2Q_WAVE;
    const int ntt = (T + kPfTile - 1) / kPfTile;
    const int ntg = (ntt + NT - 1) / NT;
    const int nrt = (rows + kPfTile - 1) / kPfTile;
    if (gw >= nrt * ntg) return;   // wave-uniform: no barrier follows
    const int rt = gw / ntg, tg = gw - rt * ntg;
    const int nb = cols / G;
    const int kq = lane / 16;
    constexpr int CH = G / 4;
    const int ra = min(rt * kPfTile + lane % 16, rows - 1);       // A row of this lane
    const uint8_t* wrow = w + (size_t)ra * cols * BITS / 8;
    int tb[NT];                                                   // B / D token of this lane per tile
#pragma unroll
    for (int j = 0; j < NT; j++) tb[j] = min((tg * NT + j) * kPfTile + lane % 16, T - 1);
    size_t wsrow[4];                                              // D rows of this lane
#pragma unroll
    for (int i = 0; i < 4; i++) wsrow[i] = (size_t)min(rt * kPfTile + 4 * kq + i, rows - 1) * nb;

    auto load = [&](int b, PfOperands<BITS, G, NT>& o) {
        pf_load_a<BITS, G>(wrow, b, kq, o.a);
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int* xp = reinterpret_cast<const int*>(xqp + (size_t)tb[j] * cols + (size_t)b * G + kq * CH);
#pragma unroll
            for (int v = 0; v < G / 16; v++) o.bx[j][v] = xp[v];
            const size_t gi = (size_t)tb[j] * nb + b;
            o.gxs[j] = xs[gi];
            o.gxt[j] = xt[gi];
            o.gsq[j] = sq[gi];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) o.ws4[i] = ws[wsrow[i] + b];
    };
    float acc[NT][4];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = 0.0f;
    auto fold = [&](const PfOperands<BITS, G, NT>& o) {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            v4i32 d4 = {0, 0, 0, 0};
            if constexpr (G == 64) {
                const v4i32 av = {o.a[0], o.a[1], o.a[2], o.a[3]};
                const v4i32 bv = {o.bx[j][0], o.bx[j][1], o.bx[j][2], o.bx[j][3]};
                d4 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, d4, 0, 0, 0);
            } else {
                const long av = (long)(unsigned)o.a[0] | ((long)o.a[1] << 32);
                const long bv = (long)(unsigned)o.bx[j][0] | ((long)o.bx[j][1] << 32);
                d4 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, d4, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d = BITS == 4 ? d4[i] >> 4 : d4[i];   // exact: the x16 dot is a multiple of 16
                acc[j][i] = __builtin_fmaf(o.ws4[i], group_term(o.gxs[j], o.gxt[j], d, o.gsq[j]), acc[j][i]);
            }
        }
    };
    PfOperands<BITS, G, NT> s0, s1;
    load(0, s0);
    for (int b = 0; b < nb; b += 2) {
        load(min(b + 1, nb - 1), s1);
        fold(s0);
        load(min(b + 2, nb - 1), s0);
        if (b + 1 < nb) fold(s1);
    }
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const int t = (tg * NT + j) * kPfTile + lane % 16;
        if (t < T) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rt * kPfTile + 4 * kq + i;
                if (r < rows) out[(size_t)t * ldo + r] = acc[j][i];
            }
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
// h13 [T][2n] -> xq [T][n], xs [T][n/G], as k_swiglu_quant per token.
template <int G>
__global__ __launch_bounds__(256) void k_pf_swiglu_quant(const float* __restrict__ h13, int n, int T,
                                                         int8_t* __restrict__ xq, float* __restrict__ xs) {
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
    if (in) {
        xq[i] = (int8_t)q8_value_fast(g, s, q8_recip(s));
        if ((i % G) == 0) xs[i / G] = s;
    }
}

}  // namespace l2q
