// kernels.h - the non-GEMV decode kernels: Q8 quantize, fused residual +
// RMSNorm + quantize, SwiGLU + quantize, RoPE + KV append, split-context
// single-query attention and the device argmax.
//
// Positions: kernels used inside the captured decode graph read the token
// and position from device memory (`meta` = {token, pos}), so one graph
// serves every step; the op ABI passes them by value (meta == NULL).
#pragma once
#include "device.h"
#include "exp_runq.h"
#include "gemv.h"

namespace l2q {

__device__ __forceinline__ int meta_pos(const int* meta, int pos) { return meta ? meta[1] : pos; }

// ---------------------------------------------------------------------------
// Q8 quantize (runq.c:117-139).  One thread per element, groups of G
// consecutive lanes (G divides 64, so a group never straddles a wave).
// pf.xqp set: also the prefill GEMM operand (pf_emit); xq may then be null.
template <int G>
__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ x, int n,
                                                  int8_t* __restrict__ xq, float* __restrict__ xs, PfOperand pf) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool in = i < n;
    const float v = in ? x[i] : 0.0f;
    const float s = q8_scale(group_max<G>(fabsf(v)));
    const int q = q8_value_fast(v, s, q8_recip(s));
    if (pf.xqp) {
        const int t = i / pf.K;
        pf_emit<G>(pf, t, i - t * pf.K, q, s, in);
    }
    if (in) {
        if (xq) xq[i] = (int8_t)q;
        if (xs && (i % G) == 0) xs[i / G] = s;
    }
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm + Q8 quantize of one vector (runq.c:294-305 then
// :117-139; the residual fold of v5-cuda-fused/run.cu:120-175).  One
// workgroup of 1024 threads; element i is owned by thread i % 1024, so each
// wave holds 64 consecutive elements and groups stay inside a wave.
// If `emb` is set, x is the embedding row of the token in meta[0].
//
// The sum of squares follows the reference's order exactly: 16 lanes each
// accumulate x[j]*x[j] with FMA over j = l, l+16, ... (its AVX-512 loop),
// the 16 partials are reduced pairwise (8, 4, then (0,2)+(1,3)) as
// _mm512_reduce_add_ps does, and a tail of n % 16 elements is added the way
// GCC compiles the reference's scalar loop (a block of 8 unfused, then
// FMAs).  So inv, and every quantized activation, is bit-identical.
template <int G>
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm_quant(
    const float* __restrict__ x, const float* __restrict__ emb, const int* __restrict__ meta,
    const float* __restrict__ resid, float* __restrict__ xout, const float* __restrict__ w, int n,
    int8_t* __restrict__ xq, float* __restrict__ xs) {
    __shared__ float vs[kNormThreads * kNormMaxPer];
    __shared__ float inv_s;
    const int tid = threadIdx.x;
    // workgroup t normalises vector t of a batch (rows of n; one vector per launch on the decode path)
    const size_t to = (size_t)blockIdx.x * n;
    if (blockIdx.x) {
        x += to;
        if (resid) resid += to;
        if (xout) xout += to;
        xq += to;
        xs += to / G;
    }
    const float* src = emb ? emb + (size_t)meta[0] * n : x;
    float v[kNormMaxPer], wv[kNormMaxPer];
#pragma unroll
    for (int k = 0; k < kNormMaxPer; k++) {
        const int i = tid + k * kNormThreads;
        float t = 0.0f;
        if (i < n) {
            t = src[i];
            if (resid) t += resid[i];
            vs[i] = t;
        }
        v[k] = t;
        wv[k] = i < n ? w[i] : 0.0f;   // the norm weights ride with the inputs: one round trip, not two
    }
    __syncthreads();
    if (tid < L2Q_WAVE) {
        const float ss = runq_sumsq(vs, n, tid);
        if (tid == 0) inv_s = 1.0f / sqrtf(ss / (float)n + 1e-5f);
    }
    __syncthreads();
    const float inv = inv_s;
#pragma unroll
    for (int k = 0; k < kNormMaxPer; k++) {
        const int i = tid + k * kNormThreads;
        if (k * kNormThreads >= n) break;   // uniform across the workgroup
        const bool in = i < n;
        const float o = in ? wv[k] * (inv * v[k]) : 0.0f;
        const float s = q8_scale(group_max<G>(fabsf(o)));
        const int q = q8_value_fast(o, s, q8_recip(s));
        if (in) {
            if (xout) xout[i] = v[k];
            xq[i] = (int8_t)q;
            if ((i % G) == 0) xs[i / G] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// SwiGLU + Q8 quantize (runq.c:404-412):  g = (h * (1/(1+expf(-h)))) * h2.
template <int G>
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* __restrict__ hb,
                                                      const float* __restrict__ hb2, int n,
                                                      int8_t* __restrict__ xq, float* __restrict__ xs,
                                                      float* __restrict__ gout) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool in = i < n;
    float g = 0.0f;
    if (in) {
        float h = hb[i];
        h *= (1.0f / (1.0f + exp_runq(-h)));
        g = h * hb2[i];
    }
    const float s = q8_scale(group_max<G>(fabsf(g)));
    if (in) {
        xq[i] = (int8_t)q8_value_fast(g, s, q8_recip(s));
        if ((i % G) == 0) xs[i / G] = s;
        if (gout) gout[i] = g;
    }
}

// ---------------------------------------------------------------------------
// RoPE + KV append (runq.c:340-365).  One thread per (even, odd) pair of
// the query; pairs inside kv_dim also rotate k and store k, v at `pos`.
// The (cos, sin) come from the host-built table (bit-identical to libm).
// Rotation as a GCC -O3 -march=native build of the reference evaluates it:
//   v0' = fma(v0, c, -(v1*s)),  v1' = fma(v0, s, v1*c).
// Cache layout [n_kv_heads][max_t][head_size] (V; K as k_index with k_il).
// Workgroup row y handles token y of a batch at position pos + y, its q, k,
// v rows `stride` floats after the previous token's (prefill).
__global__ __launch_bounds__(256) void k_rope_kv_append(
    float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ kcache, float* __restrict__ vcache, const float* __restrict__ rope,
    const int* __restrict__ meta, int pos_arg, int dim, int kv_dim, int hs, int max_t, int stride, int k_il) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    const int i = 2 * p;
    if (i >= dim) return;
    const int pos = meta_pos(meta, pos_arg) + blockIdx.y;
    q += (size_t)blockIdx.y * stride;
    k += (size_t)blockIdx.y * stride;
    v += (size_t)blockIdx.y * stride;
    const int hd = i % hs;
    const float c = rope[(size_t)pos * hs + hd];
    const float s = rope[(size_t)pos * hs + hd + 1];
    {
        const float v0 = q[i], v1 = q[i + 1];
        q[i] = __builtin_fmaf(v0, c, -(v1 * s));
        q[i + 1] = __builtin_fmaf(v0, s, v1 * c);
    }
    if (i < kv_dim) {
        const int h = i / hs;
        const size_t off = ((size_t)h * max_t + pos) * hs + hd;
        const size_t ko = k_index(k_il, h, pos, hd, hs, max_t);   // hd even: hd, hd + 1 share a float4
        const float k0 = k[i], k1 = k[i + 1];
        kcache[ko] = __builtin_fmaf(k0, c, -(k1 * s));
        kcache[ko + 1] = __builtin_fmaf(k0, s, k1 * c);
        vcache[off] = v[i];
        vcache[off + 1] = v[i + 1];
    }
}

// ---------------------------------------------------------------------------
// Single-query attention, split over the context (runq.c:367-391 +
// softmax :307-318; the tolerance path of BASELINE config 4).  Workgroup
// (head h, split s) covers positions [s*C, min((s+1)*C, pos+1)) with C =
// ceil((pos+1)/S):
//   scores   four lanes per position (lane sub sums the 4-element chunks
//            4*sub + 16*i with FMAs, K read straight from the cache as
//            float4, q held in registers), 64 positions per pass, all of a
//            pass's loads in flight at once; scores to LDS;
//   softmax  block max m and l = sum_t exp(s_t - m) over the split;
//   p*V      thread (slice, g) accumulates elements 4g..4g+3 (float4 loads,
//            a 512 B row per 32 threads) over positions t = slice (mod
//            slices), four rows in flight; the slices are added in LDS.
// It leaves the partial (m, l, o[hs]) with o unnormalised; k_attn_combine
// merges the S partials of a head.
__host__ __device__ constexpr size_t attn_lds_bytes(int C, int hs) {
    return ((size_t)(C + 3) / 4 * 4 + 4 * kAttnThreads + 16) * sizeof(float);
}

__global__ __launch_bounds__(kAttnThreads) void k_attn_partial(
    const float* __restrict__ q, const float* __restrict__ kcache, const float* __restrict__ vcache,
    float* __restrict__ part_o, float* __restrict__ part_ml, const int* __restrict__ meta, int pos_arg,
    int n_heads, int kv_mul, int hs, int max_t) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int h = blockIdx.x, s = blockIdx.y, S = gridDim.y;
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE, sub = tid & 3;
    const int pos = meta_pos(meta, pos_arg);
    const int n = pos + 1;
    const int C = (n + S - 1) / S;
    const int t0 = min(s * C, n), t1 = min(n, t0 + C);
    float* sc = smem;                                   // [C] scores, then exp(s - m)
    float* part = sc + (C + 3) / 4 * 4;                 // [slices][hs]
    float* red = part + 4 * kAttnThreads;               // [8] block reductions
    float* po = part_o + ((size_t)h * S + s) * hs;
    float* pml = part_ml + ((size_t)h * S + s) * 2;
    if (t0 >= t1) {   // empty split (uniform across the workgroup)
        for (int d = tid; d < hs; d += kAttnThreads) po[d] = 0.0f;
        if (tid == 0) { pml[0] = -INFINITY; pml[1] = 0.0f; }
        return;
    }
    const int kvh = h / kv_mul;
    const float* kbase = kcache + (size_t)kvh * max_t * hs;
    const float* vbase = vcache + (size_t)kvh * max_t * hs;
    const float* qh = q + (size_t)h * hs;
    constexpr int kQChunks = kAttnMaxHs / 16;           // float4 chunks of q per lane (hs <= 256)
    float4 qr[kQChunks];
#pragma unroll
    for (int i = 0; i < kQChunks; i++)
        qr[i] = 16 * i + 4 * sub < hs ? *reinterpret_cast<const float4*>(qh + 16 * i + 4 * sub)
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float rs = sqrtf((float)hs);
    for (int tb = t0; tb < t1; tb += kAttnThreads / 4) {
        const int t = tb + tid / 4;
        const float* kr = kbase + (size_t)min(t, t1 - 1) * hs;
        float4 kk[kQChunks];
#pragma unroll
        for (int i = 0; i < kQChunks; i++)
            kk[i] = 16 * i + 4 * sub < hs ? *reinterpret_cast<const float4*>(kr + 16 * i + 4 * sub)
                                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kQChunks; i++) {
            if (16 * i < hs) {
                acc = __builtin_fmaf(qr[i].x, kk[i].x, acc);
                acc = __builtin_fmaf(qr[i].y, kk[i].y, acc);
                acc = __builtin_fmaf(qr[i].z, kk[i].z, acc);
                acc = __builtin_fmaf(qr[i].w, kk[i].w, acc);
            }
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        if (sub == 0 && t < t1) sc[t - t0] = acc / rs;
    }
    __syncthreads();
    const int m_n = t1 - t0;
    float m = -INFINITY;
    for (int j = tid; j < m_n; j += kAttnThreads) m = fmaxf(m, sc[j]);
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
    for (int j = tid; j < m_n; j += kAttnThreads) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        l += e;
    }
    l = wave_sum(l);
    if (lane == 0) red[4 + wv] = l;
    __syncthreads();
    l = (red[4] + red[5]) + (red[6] + red[7]);
    const int groups = hs / 4, slices = kAttnThreads / groups;
    const int gi = tid % groups, slice = tid / groups;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (slice < slices) {
        const float* vb = vbase + 4 * gi;
#pragma unroll 4
        for (int j = slice; j < m_n; j += slices) {
            const float4 vv = *reinterpret_cast<const float4*>(vb + (size_t)(t0 + j) * hs);
            const float p = sc[j];
            o.x = __builtin_fmaf(p, vv.x, o.x);
            o.y = __builtin_fmaf(p, vv.y, o.y);
            o.z = __builtin_fmaf(p, vv.z, o.z);
            o.w = __builtin_fmaf(p, vv.w, o.w);
        }
        *reinterpret_cast<float4*>(part + (size_t)slice * hs + 4 * gi) = o;
    }
    __syncthreads();
    for (int d = tid; d < hs; d += kAttnThreads) {
        float t = 0.0f;
        for (int k = 0; k < slices; k++) t += part[(size_t)k * hs + d];
        po[d] = t;
    }
    if (tid == 0) { pml[0] = m; pml[1] = l; }
}

// ---------------------------------------------------------------------------
// Attention in the reference's exact order (runq.c:367-391, softmax
// :307-318), in two kernels:
//
// k_attn_scores: one workgroup per work item (head h, tile of kScoreTile
//   positions), persistent over the items of the current position: the K
//   rows of the tile are staged in LDS with coalesced 128-bit loads (all in
//   flight at once), then one lane per position forms
//   sum_i q_i*k_i over the head in index order
//   (products rounded, added in order - GCC vectorises the reference loop
//   that way; a remainder of head_size % 8 is fused), then / sqrtf(hs).
// k_attn_softmax_v: workgroup (head h, kVDims output elements) takes the
//   max of the head's scores, e_t = expf(s_t - max) with the host-identical
//   exp_runq, the sum of e_t in position order (one lane), p_t = e_t / sum,
//   and then one lane per output element accumulates fma(p_t, v_t[i], acc)
//   in position order.  V is streamed through LDS in chunks of kVChunk
//   positions, transposed to [element][position] so that each chain reads
//   four positions per LDS load; both serial chains read their operands a
//   block ahead of the FMAs, and the next V chunk's loads are in flight
//   while the current chunk is folded.
constexpr int kScoreTile = 16;
constexpr int kScoreThreads = L2Q_WAVE;
constexpr int kScoreGridMax = 1024;
constexpr int kVDims = 16;
constexpr int kVChunk = 256;
constexpr int kVStride = kVChunk + 4;                              // LDS row of one element's chunk
constexpr int kVPer = kVChunk * kVDims / 4 / kAttnThreads;         // float4 per thread per chunk
constexpr int kScorePer = 16;                                      // scores per thread -> n <= 4096

// (+ kRingSlack floats: the serial chains' ring reads run up to 24 floats
// past their arrays)
constexpr int kRingSlack = 32;
__host__ __device__ constexpr size_t attn_scores_lds_bytes(int hs) {
    return ((size_t)kScoreTile * (hs + 4) + hs + kRingSlack) * sizeof(float);
}
__host__ __device__ constexpr size_t attn_v_lds_bytes(int max_t) {
    return ((size_t)(max_t + 7) / 4 * 4 + 2 * kVDims * kVStride + 8 + kRingSlack) * sizeof(float);
}

// q.k over a head in the reference's order: products rounded, added in
// index order for the first hs & ~7 elements, the rest fused (k and q in
// LDS, 16-byte aligned).  k streams through a ring of R float4 blocks, each
// loaded R-1 blocks ahead of the adds; loads may run up to R blocks past
// the row (inside the workgroup's LDS), never added.
template <int R = 6>
__device__ __forceinline__ float serial_dot(const float* kr, const float* qs, int hs) {
#pragma clang fp contract(off)
    const float4* k4 = reinterpret_cast<const float4*>(kr);
    const float4* q4 = reinterpret_cast<const float4*>(qs);
    const int nv = (hs & ~7) >> 2;   // float4 blocks added unfused
    float4 K[R], Q[R];
#pragma unroll
    for (int j = 0; j < R; j++) { K[j] = k4[j]; Q[j] = q4[j]; }
    float score = 0.0f;
    int b = 0;
    for (; b + R <= nv; b += R) {
#pragma unroll
        for (int j = 0; j < R; j++) {
            score = score + Q[j].x * K[j].x;
            score = score + Q[j].y * K[j].y;
            score = score + Q[j].z * K[j].z;
            score = score + Q[j].w * K[j].w;
            __builtin_amdgcn_sched_barrier(0);
            K[j] = k4[b + j + R];
            Q[j] = q4[b + j + R];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int j = 0; j < R; j++) {
        if (b + j < nv) {
            score = score + Q[j].x * K[j].x;
            score = score + Q[j].y * K[j].y;
            score = score + Q[j].z * K[j].z;
            score = score + Q[j].w * K[j].w;
        }
    }
    for (int i = nv * 4; i < hs; i++) score = __builtin_fmaf(qs[i], kr[i], score);
    return score;
}

// Grid row y: query y of a batch at position pos + y, its q `q_stride`
// floats after the previous query's, scores in its own [n_heads][max_t].
__global__ __launch_bounds__(kScoreThreads) void k_attn_scores(
    const float* __restrict__ q, const float* __restrict__ kcache, float* __restrict__ scores,
    const int* __restrict__ meta, int pos_arg, int kv_mul, int n_heads, int hs, int max_t, int q_stride, int k_il) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int hsp = hs + 4;
    float* kt = sm;                       // [kScoreTile][hsp]
    float* qs = kt + kScoreTile * hsp;    // [hs]
    const int tid = threadIdx.x;
    const int pos = meta_pos(meta, pos_arg) + blockIdx.y;
    q += (size_t)blockIdx.y * q_stride;
    scores += (size_t)blockIdx.y * n_heads * max_t;
    const int n = pos + 1;
    const int ntile = (n + kScoreTile - 1) / kScoreTile;
    const int f4 = hs / 4;
    for (int item = blockIdx.x; item < n_heads * ntile; item += gridDim.x) {
        const int h = item / ntile;
        const int t0 = (item - h * ntile) * kScoreTile;
        const int nt = min(kScoreTile, n - t0);
        const int g = h / kv_mul;
        // the tile's loads in batches of 8 float4 per lane, all of a batch in
        // flight at once (one batch covers a 16 x 128 tile); consecutive
        // lanes read consecutive float4 of the cache in either layout
        auto tile_rc = [&](int f, int& r, int& c4) {
            if (k_il) { c4 = f / nt; r = f - c4 * nt; }
            else { r = f / f4; c4 = f - r * f4; }
        };
        for (int b0 = 0; b0 < nt * f4; b0 += 8 * kScoreThreads) {
            float4 kv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                int r, c4;
                tile_rc(min(b0 + tid + kScoreThreads * k, nt * f4 - 1), r, c4);
                kv[k] = *reinterpret_cast<const float4*>(kcache + k_index(k_il, g, t0 + r, 4 * c4, hs, max_t));
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int f = b0 + tid + kScoreThreads * k;
                if (f < nt * f4) {
                    int r, c4;
                    tile_rc(f, r, c4);
                    *reinterpret_cast<float4*>(kt + r * hsp + 4 * c4) = kv[k];
                }
            }
        }
        for (int d = tid; d < hs; d += kScoreThreads) qs[d] = q[(size_t)h * hs + d];
        __syncthreads();
        if (tid < nt) scores[(size_t)h * max_t + t0 + tid] = serial_dot(kt + tid * hsp, qs, hs) / sqrtf((float)hs);
        __syncthreads();   // the next item restages the tile
    }
}

// Sequential sum of p[0..n) (p 16-byte aligned in LDS), non-fused adds in
// index order.  p streams through a ring of R float4 blocks loaded R-1
// blocks ahead of the adds (reads may run R blocks past p[n), inside the
// workgroup's LDS, never added).
template <int R = 6>
__device__ __forceinline__ float serial_sum(const float* p, int n) {
#pragma clang fp contract(off)
    const float4* p4 = reinterpret_cast<const float4*>(p);
    const int nb = n >> 2;
    float4 P[R];
#pragma unroll
    for (int j = 0; j < R; j++) P[j] = p4[j];
    float sum = 0.0f;
    int b = 0;
    for (; b + R <= nb; b += R) {
#pragma unroll
        for (int j = 0; j < R; j++) {
            sum = sum + P[j].x; sum = sum + P[j].y; sum = sum + P[j].z; sum = sum + P[j].w;
            __builtin_amdgcn_sched_barrier(0);
            P[j] = p4[b + j + R];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int j = 0; j < R; j++)
        if (b + j < nb) { sum = sum + P[j].x; sum = sum + P[j].y; sum = sum + P[j].z; sum = sum + P[j].w; }
    for (int t = nb * 4; t < n; t++) sum = sum + p[t];
    return sum;
}

// acc = fma(p[t], v[t], acc) for t = 0..n-1 in order (both 16-byte aligned
// in LDS), through a ring of R float4 blocks of each (as serial_sum).
template <int R = 6>
__device__ __forceinline__ float serial_pv(const float* p, const float* v, int n, float acc) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    const float4* v4 = reinterpret_cast<const float4*>(v);
    const int nb = n >> 2;
    float4 P[R], V[R];
#pragma unroll
    for (int j = 0; j < R; j++) { P[j] = p4[j]; V[j] = v4[j]; }
    int b = 0;
    for (; b + R <= nb; b += R) {
#pragma unroll
        for (int j = 0; j < R; j++) {
            acc = __builtin_fmaf(P[j].x, V[j].x, acc);
            acc = __builtin_fmaf(P[j].y, V[j].y, acc);
            acc = __builtin_fmaf(P[j].z, V[j].z, acc);
            acc = __builtin_fmaf(P[j].w, V[j].w, acc);
            __builtin_amdgcn_sched_barrier(0);
            P[j] = p4[b + j + R];
            V[j] = v4[b + j + R];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int j = 0; j < R; j++) {
        if (b + j < nb) {
            acc = __builtin_fmaf(P[j].x, V[j].x, acc);
            acc = __builtin_fmaf(P[j].y, V[j].y, acc);
            acc = __builtin_fmaf(P[j].z, V[j].z, acc);
            acc = __builtin_fmaf(P[j].w, V[j].w, acc);
        }
    }
    for (int t = nb * 4; t < n; t++) acc = __builtin_fmaf(p[t], v[t], acc);
    return acc;
}

// Grid z: query z of a batch (position pos + z, scores and output of its own).
__global__ __launch_bounds__(kAttnThreads) void k_attn_softmax_v(
    const float* __restrict__ scores, const float* __restrict__ vcache, float* __restrict__ out,
    const int* __restrict__ meta, int pos_arg, int kv_mul, int hs, int max_t) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* p = smem;                                     // [max_t] probabilities
    float* vt = smem + (max_t + 7) / 4 * 4;              // [2][kVDims][kVStride]
    float* red = vt + 2 * kVDims * kVStride;             // [4] wave maxima, [4] sum
    const int h = blockIdx.x, d0 = blockIdx.y * kVDims;
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE;
    const int pos = meta_pos(meta, pos_arg) + blockIdx.z;
    const int n = pos + 1;
    const int width = min(kVDims, hs - d0);
    scores += (size_t)blockIdx.z * gridDim.x * max_t;
    out += (size_t)blockIdx.z * gridDim.x * hs;
    const float* sc = scores + (size_t)h * max_t;
    const float* vbase = vcache + (size_t)(h / kv_mul) * max_t * hs + d0;
    const int nchunks = (n + kVChunk - 1) / kVChunk;

    // scores first, then the first V chunk (loads complete in order)
    float s[kScorePer];
#pragma unroll
    for (int k = 0; k < kScorePer; k++) {
        const int t = tid + kAttnThreads * k;
        s[k] = t < n ? sc[t] : -INFINITY;
    }
    float4 vr[kVPer];
    auto load_chunk = [&](int c) {
#pragma unroll
        for (int k = 0; k < kVPer; k++) {
            const int e = tid + kAttnThreads * k;                 // float4 index in the chunk
            const int r = e / (kVDims / 4), c4 = e % (kVDims / 4);
            const int t = c * kVChunk + r;
            vr[k] = (t < n && 4 * c4 < width) ? *reinterpret_cast<const float4*>(vbase + (size_t)t * hs + 4 * c4)
                                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto store_chunk = [&](int buf) {   // transposed: vt[buf][element][position]
        float* dst = vt + buf * kVDims * kVStride;
#pragma unroll
        for (int k = 0; k < kVPer; k++) {
            const int e = tid + kAttnThreads * k;
            const int r = e / (kVDims / 4), c4 = e % (kVDims / 4);
            dst[(4 * c4 + 0) * kVStride + r] = vr[k].x;
            dst[(4 * c4 + 1) * kVStride + r] = vr[k].y;
            dst[(4 * c4 + 2) * kVStride + r] = vr[k].z;
            dst[(4 * c4 + 3) * kVStride + r] = vr[k].w;
        }
    };
    load_chunk(0);

    // softmax in the reference's order
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kScorePer; k++) m = fmaxf(m, s[k]);
    m = group_max<L2Q_WAVE>(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float e[kScorePer];
#pragma unroll
    for (int k = 0; k < kScorePer; k++) {
        const int t = tid + kAttnThreads * k;
        e[k] = 0.0f;
        if (kAttnThreads * k < n && t < n) {   // the first test is uniform: skips whole rounds
            e[k] = exp_runq(s[k] - m);
            p[t] = e[k];
        }
    }
    __syncthreads();
    if (tid == 0) red[4] = serial_sum(p, n);
    __syncthreads();
    const float sum = red[4];
#pragma unroll
    for (int k = 0; k < kScorePer; k++) {
        const int t = tid + kAttnThreads * k;
        if (kAttnThreads * k < n && t < n) p[t] = e[k] / sum;
    }
    store_chunk(0);
    __syncthreads();

    // serial p*V chains, one lane per output element, V double-buffered in LDS
    float acc = 0.0f;
    for (int c = 0; c < nchunks; c++) {
        if (c + 1 < nchunks) load_chunk(c + 1);
        if (wv == 0 && lane < width) {
            const int tb = c * kVChunk;
            acc = serial_pv(p + tb, vt + (c & 1) * kVDims * kVStride + lane * kVStride, min(kVChunk, n - tb), acc);
        }
        if (c + 1 < nchunks) store_chunk((c + 1) & 1);
        __syncthreads();
    }
    if (wv == 0 && lane < width) out[(size_t)h * hs + d0 + lane] = acc;
}

// ---------------------------------------------------------------------------
// Batched attention (T > 1 queries at positions pos..pos+T-1, causal), the
// same operations in the same order as k_attn_scores + k_attn_softmax_v, so
// every output is bit-identical to T single-query steps; three kernels that
// share each K and V row over the queries instead of re-reading it per query.
//
// k_attn_scores_b: workgroup (head, 64-key tile, 32-query block): the K tile
//   and the block's q rows are staged in LDS once; thread (key t, query group
//   g) forms the dots of key t with queries 8g..8g+7 (eight independent
//   chains), each in serial_dot's order (products rounded and added in index
//   order over hs & ~7 elements, the rest fused), / sqrtf(hs); pairs above
//   the causal diagonal are skipped.
constexpr int kSbKeys = 64, kSbQueries = 32, kSbThreads = 256;
constexpr int kSbPer = kSbQueries * kSbKeys / kSbThreads;   // chains per thread (8)
__host__ __device__ constexpr size_t attn_scores_b_lds_bytes(int hs) {
    return (size_t)(kSbKeys + kSbQueries) * (hs + 4) * sizeof(float);
}
__global__ __launch_bounds__(kSbThreads) void k_attn_scores_b(
    const float* __restrict__ q, const float* __restrict__ kcache, float* __restrict__ scores, int pos0, int T,
    int kv_mul, int n_heads, int hs, int max_t, int q_stride, int k_il) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int hsp = hs + 4;
    float* kt = sm;                      // [kSbKeys][hsp]
    float* qs = kt + kSbKeys * hsp;      // [kSbQueries][hsp]
    const int h = blockIdx.x, t0 = blockIdx.y * kSbKeys, q0 = blockIdx.z * kSbQueries;
    const int tid = threadIdx.x;
    const int nk = pos0 + T;
    // the tile's first key is past the block's last query's position: no pair
    if (t0 > pos0 + min(q0 + kSbQueries, T) - 1) return;
    const int g = h / kv_mul, f4 = hs / 4;
    const int nt = min(kSbKeys, nk - t0);
    // the tile's and the q block's loads in batches of four per thread, all
    // of a batch in flight before its stores (clamped indices; a load per
    // iteration followed by its store would wait one memory latency each)
    const int nkf = kSbKeys * f4, nqf = kSbQueries * f4;
    auto k_addr = [&](int f, int& r, int& c4) {
        f = min(f, nkf - 1);
        if (k_il) { c4 = f / kSbKeys; r = f - c4 * kSbKeys; }   // consecutive lanes, consecutive keys
        else { r = f / f4; c4 = f - r * f4; }
        return reinterpret_cast<const float4*>(kcache + k_index(k_il, g, t0 + min(r, nt - 1), 4 * c4, hs, max_t));
    };
    for (int b = 0; b < nkf; b += 4 * kSbThreads) {
        int r0, c0, r1, c1, r2, c2, r3, c3;
        const float4 v0 = *k_addr(b + tid, r0, c0), v1 = *k_addr(b + tid + kSbThreads, r1, c1);
        const float4 v2 = *k_addr(b + tid + 2 * kSbThreads, r2, c2), v3 = *k_addr(b + tid + 3 * kSbThreads, r3, c3);
        if (b + tid < nkf) *reinterpret_cast<float4*>(kt + r0 * hsp + 4 * c0) = v0;
        if (b + tid + kSbThreads < nkf) *reinterpret_cast<float4*>(kt + r1 * hsp + 4 * c1) = v1;
        if (b + tid + 2 * kSbThreads < nkf) *reinterpret_cast<float4*>(kt + r2 * hsp + 4 * c2) = v2;
        if (b + tid + 3 * kSbThreads < nkf) *reinterpret_cast<float4*>(kt + r3 * hsp + 4 * c3) = v3;
    }
    auto q_addr = [&](int f) {
        f = min(f, nqf - 1);
        return reinterpret_cast<const float4*>(q + (size_t)min(q0 + f / f4, T - 1) * q_stride + (size_t)h * hs +
                                               4 * (f % f4));
    };
    for (int b = 0; b < nqf; b += 4 * kSbThreads) {
        const float4 v0 = *q_addr(b + tid), v1 = *q_addr(b + tid + kSbThreads);
        const float4 v2 = *q_addr(b + tid + 2 * kSbThreads), v3 = *q_addr(b + tid + 3 * kSbThreads);
        const float4 vv[4] = {v0, v1, v2, v3};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int f = b + tid + k * kSbThreads;
            if (f < nqf) *reinterpret_cast<float4*>(qs + (f / f4) * hsp + 4 * (f % f4)) = vv[k];
        }
    }
    __syncthreads();
    const int tl = tid % kSbKeys, qg = tid / kSbKeys;
    const float4* k4 = reinterpret_cast<const float4*>(kt + tl * hsp);
    float sc[kSbPer];
#pragma unroll
    for (int j = 0; j < kSbPer; j++) sc[j] = 0.0f;
    const int nv = (hs & ~7) >> 2;   // float4 blocks added unfused, then the fused rest
    const float4* qb = reinterpret_cast<const float4*>(qs + qg * kSbPer * hsp);
    const int qp = hsp / 4;          // q row pitch in float4
    for (int c = 0; c < nv; c++) {
        // the step's LDS reads issued together, then the adds
        const float4 kv = k4[c];
        float4 qv[kSbPer];
#pragma unroll
        for (int j = 0; j < kSbPer; j++) qv[j] = qb[j * qp + c];
#pragma unroll
        for (int j = 0; j < kSbPer; j++) {
            sc[j] = sc[j] + qv[j].x * kv.x;
            sc[j] = sc[j] + qv[j].y * kv.y;
            sc[j] = sc[j] + qv[j].z * kv.z;
            sc[j] = sc[j] + qv[j].w * kv.w;
        }
    }
    for (int c = nv; c < f4; c++) {
        const float4 kv = k4[c];
        float4 qv[kSbPer];
#pragma unroll
        for (int j = 0; j < kSbPer; j++) qv[j] = qb[j * qp + c];
#pragma unroll
        for (int j = 0; j < kSbPer; j++) {
            sc[j] = __builtin_fmaf(qv[j].x, kv.x, sc[j]);
            sc[j] = __builtin_fmaf(qv[j].y, kv.y, sc[j]);
            sc[j] = __builtin_fmaf(qv[j].z, kv.z, sc[j]);
            sc[j] = __builtin_fmaf(qv[j].w, kv.w, sc[j]);
        }
    }
    const int t = t0 + tl;
    const float rs = sqrtf((float)hs);
#pragma unroll
    for (int j = 0; j < kSbPer; j++) {
        const int qi = q0 + qg * kSbPer + j;
        if (qi < T && t < nk && t <= pos0 + qi) scores[((size_t)qi * n_heads + h) * attn_b_pitch(max_t) + t] = sc[j] / rs;
    }
}

// k_attn_softmax_b: one wave per (query, head): max, e_t = exp_runq(s_t -
// max) into LDS, the sum of e_t in position order (one lane, serial_sum),
// p_t = e_t / sum written over the scores (k_attn_softmax_v's softmax).
constexpr int kSmThreads = L2Q_WAVE;
__host__ __device__ constexpr size_t attn_softmax_b_lds_bytes(int max_t) {
    return ((size_t)(max_t + 3) / 4 * 4 + kRingSlack + 4) * sizeof(float);
}
__global__ __launch_bounds__(kSmThreads) void k_attn_softmax_b(float* __restrict__ scores, int pos0, int n_heads,
                                                               int max_t, int nmax) {
#pragma clang fp contract(off)
    // LDS sized for the launch's longest row, nmax = pos0 + T (not the
    // cache's max_t): more of these one-wave workgroups fit on a CU
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* p = sm;                                         // [n] e_t
    float* red = sm + (nmax + 3) / 4 * 4 + kRingSlack;     // [1] sum
    const int qi = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int n = pos0 + qi + 1;
    float* row = scores + ((size_t)qi * n_heads + h) * attn_b_pitch(max_t);
    float m = -INFINITY;
    for (int t0 = 0; t0 < n; t0 += 8 * kSmThreads) {   // eight loads in flight per lane
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = row[min(t0 + lane + kSmThreads * k, n - 1)];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int t = t0 + lane + kSmThreads * k;
            if (t < n) {
                p[t] = v[k];
                m = fmaxf(m, v[k]);
            }
        }
    }
    m = group_max<L2Q_WAVE>(m);
    for (int t = lane; t < n; t += kSmThreads) p[t] = exp_runq(p[t] - m);
    __syncthreads();
    if (lane == 0) red[0] = serial_sum(p, n);
    __syncthreads();
    const float sum = red[0];
    for (int t = lane; t < n; t += kSmThreads) row[t] = p[t] / sum;
}

// k_attn_pv_b: workgroup (head, 16-element slice, 128-query block): thread
// (query ql, element quad) accumulates acc_i = fma(p_t, v_t[i], acc_i) over
// t = 0..pos+ql in position order for four elements (k_attn_softmax_v's
// serial_pv), over 64-key chunks of V and of the block's p rows staged in
// LDS, the next chunk's loads in flight while the current one is folded.
constexpr int kPvKeys = 64, kPvQueries = 128, kPvThreads = 512;
constexpr int kPvPitch = kPvKeys + 1;   // odd: the 16 queries of a wave read distinct banks
__global__ __launch_bounds__(kPvThreads) void k_attn_pv_b(const float* __restrict__ p, const float* __restrict__ vcache,
                                                          float* __restrict__ out, int pos0, int T, int kv_mul,
                                                          int n_heads, int hs, int max_t) {
    __shared__ float pt[kPvQueries * kPvPitch];
    __shared__ float4 vt[kPvKeys][kVDims / 4];
    const int h = blockIdx.x, d0 = blockIdx.y * kVDims, q0 = blockIdx.z * kPvQueries;
    const int tid = threadIdx.x, ql = tid >> 2, quad = tid & 3;
    const int width = min(kVDims, hs - d0);
    const int qi = q0 + ql;
    const int n = qi < T ? pos0 + qi + 1 : 0;              // keys of this thread's query
    const int nblk = pos0 + min(q0 + kPvQueries, T);       // keys of the block's last query
    const int nchunks = (nblk + kPvKeys - 1) / kPvKeys;
    const float* vb = vcache + (size_t)(h / kv_mul) * max_t * hs + d0;
    // staging: V row r (float4 column c4) by thread r*4 + c4 (< 256); p row
    // of query r, float4 column c4, four per thread
    constexpr int PPT = kPvQueries * kPvKeys / 4 / kPvThreads;
    float4 rv, rp[PPT];
    auto fetch = [&](int c) {
        const int t0 = c * kPvKeys;
        if (tid < kPvKeys * 4) {
            const int r = tid >> 2, c4 = tid & 3;
            rv = 4 * c4 < width ? *reinterpret_cast<const float4*>(vb + (size_t)min(t0 + r, nblk - 1) * hs + 4 * c4)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int f = tid + kPvThreads * k, r = f / (kPvKeys / 4), c4 = f % (kPvKeys / 4);
            rp[k] = *reinterpret_cast<const float4*>(p + ((size_t)min(q0 + r, T - 1) * n_heads + h) * attn_b_pitch(max_t) +
                                                     min(t0 + 4 * c4, attn_b_pitch(max_t) - 4));
        }
    };
    auto stage = [&]() {
        if (tid < kPvKeys * 4) vt[tid >> 2][tid & 3] = rv;
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int f = tid + kPvThreads * k, r = f / (kPvKeys / 4), c4 = f % (kPvKeys / 4);
            float* d = pt + r * kPvPitch + 4 * c4;
            d[0] = rp[k].x; d[1] = rp[k].y; d[2] = rp[k].z; d[3] = rp[k].w;
        }
    };
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (nchunks > 0) fetch(0);
    for (int c = 0; c < nchunks; c++) {
        stage();
        __syncthreads();
        if (c + 1 < nchunks) fetch(c + 1);
        const int tn = min(kPvKeys, n - c * kPvKeys);   // this thread's keys in the chunk
        const float* pr = pt + ql * kPvPitch;
        int t = 0;
        for (; t + 8 <= tn; t += 8) {   // a block's LDS reads issued together, then its chains
            float pv[8];
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                pv[k] = pr[t + k];
                v[k] = vt[t + k][quad];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                acc.x = __builtin_fmaf(pv[k], v[k].x, acc.x);
                acc.y = __builtin_fmaf(pv[k], v[k].y, acc.y);
                acc.z = __builtin_fmaf(pv[k], v[k].z, acc.z);
                acc.w = __builtin_fmaf(pv[k], v[k].w, acc.w);
            }
        }
        for (; t < tn; t++) {
            const float pv = pr[t];
            const float4 v = vt[t][quad];
            acc.x = __builtin_fmaf(pv, v.x, acc.x);
            acc.y = __builtin_fmaf(pv, v.y, acc.y);
            acc.z = __builtin_fmaf(pv, v.z, acc.z);
            acc.w = __builtin_fmaf(pv, v.w, acc.w);
        }
        __syncthreads();
    }
    if (qi < T && 4 * quad < width) {
        float* o = out + (size_t)qi * n_heads * hs + (size_t)h * hs + d0 + 4 * quad;
        const float a[4] = {acc.x, acc.y, acc.z, acc.w};
        for (int e = 0; e < 4 && 4 * quad + e < width; e++) o[e] = a[e];
    }
}

// k_attn_pf_b: the whole exact attention of a batch of queries whose
// context fits kPqMaxKeys (+ the Q8 quantization of its output), in one
// kernel: workgroup (head, kPqQueries-query block), HS/4 threads per query.
//   scores   the block's q rows in LDS; K in 64-key chunks through LDS (the
//            next chunk in registers while the current one is used); thread
//            (key, query group) forms its 32*64/threads dots, each in
//            k_attn_scores_b's order (products rounded and added in index
//            order over hs & ~7 elements, the rest fused, / sqrtf(hs)),
//            into the queries' LDS rows (causal pairs only);
//   softmax  the query's threads: max, e_t = exp_runq(s_t - max); one thread
//            sums e in position order (serial_sum); p_t = e_t / sum
//            (k_attn_softmax_b's operations);
//   p*V      thread (query, element quad), V staged in 64-key chunks, in
//            position order (k_attn_pv_b's);
//   out      with pf.xqp set, the wo GEMM operand: the G/4 threads of a
//            group take its max, Q8 scale and values (k_quantize's) and
//            write the permuted bytes and the record; else out [T][dim].
// Same bits as k_attn_scores_b + k_attn_softmax_b + k_attn_pv_b (+
// k_quantize), without three launches and the scores' round trip.
constexpr int kPqQueries = 16, kPqMaxKeys = 256, kPqKeys = 64;
constexpr int kPqPitch = kPqMaxKeys + 4;   // e / p rows (16-byte aligned for serial_sum)
template <int HS, int G>
__global__ __launch_bounds__(kPqQueries * HS / 4) void k_attn_pf_b(
    const float* __restrict__ q, int q_stride, const float* __restrict__ kcache, int k_il,
    const float* __restrict__ vcache, float* __restrict__ out, int pos0, int T, int kv_mul, int n_heads, int max_t,
    PfOperand pf) {
#pragma clang fp contract(off)
    constexpr int TPQ = HS / 4;                  // threads per query = element quads
    constexpr int NT = kPqQueries * TPQ;
    constexpr int HSP = HS + 4;                  // LDS row pitch of q and K (floats)
    constexpr int J = kPqQueries * kPqKeys / NT; // dot chains per thread
    constexpr int KVP = kPqKeys * TPQ / NT;      // float4 of K / V per thread per chunk
    static_assert(TPQ == 16 || TPQ == 32, "head size 64 or 128");
    static_assert(HS % G == 0, "groups inside a head");
    static_assert(KVP * NT == kPqKeys * TPQ && J * NT == kPqQueries * kPqKeys, "staging geometry");
    __shared__ __attribute__((aligned(16))) float ep[kPqQueries * kPqPitch + 4 * 8];   // + serial_sum's read-ahead
    __shared__ __attribute__((aligned(16))) float qsm[kPqQueries * HSP];
    __shared__ __attribute__((aligned(16))) float kvs[kPqKeys * HSP];                  // a K chunk, then V chunks
    __shared__ float red[kPqQueries];
    const int h = blockIdx.x, q0 = blockIdx.y * kPqQueries, g = h / kv_mul;
    const int tid = threadIdx.x, ql = tid / TPQ, quad = tid % TPQ;
    const int qi = q0 + ql;
    const int n = qi < T ? pos0 + qi + 1 : 0;                 // keys of this thread's query
    const int nblk = pos0 + min(q0 + kPqQueries, T);           // keys of the block's last query
    const int nchunks = (nblk + kPqKeys - 1) / kPqKeys;
    float* e = ep + ql * kPqPitch;
    // K: float4 f of a chunk is (key r, column c4), consecutive lanes on
    // consecutive keys with the interleaved layout (as k_attn_scores_b)
    static_assert(KVP == 4, "four float4 of K / V per thread per chunk");
    float4 kr0, kr1, kr2, kr3, vr0, vr1, vr2, vr3;   // (named: an indexed array of them went to scratch)
    // K float4 f of a chunk: (key r, column c4)
    auto kaddr = [&](int c, int f) __attribute__((always_inline)) {
        int r, c4;
        if (k_il) { c4 = f / kPqKeys; r = f - c4 * kPqKeys; }
        else { r = f / TPQ; c4 = f - r * TPQ; }
        return reinterpret_cast<const float4*>(kcache + k_index(k_il, g, min(c * kPqKeys + r, nblk - 1), 4 * c4, HS, max_t));
    };
    auto kslot = [&](int f) __attribute__((always_inline)) {
        int r, c4;
        if (k_il) { c4 = f / kPqKeys; r = f - c4 * kPqKeys; }
        else { r = f / TPQ; c4 = f - r * TPQ; }
        return reinterpret_cast<float4*>(kvs + r * HSP + 4 * c4);
    };
    auto kfetch = [&](int c) __attribute__((always_inline)) {
        kr0 = *kaddr(c, tid);
        kr1 = *kaddr(c, tid + NT);
        kr2 = *kaddr(c, tid + 2 * NT);
        kr3 = *kaddr(c, tid + 3 * NT);
    };
    auto kstore = [&]() __attribute__((always_inline)) {
        *kslot(tid) = kr0;
        *kslot(tid + NT) = kr1;
        *kslot(tid + 2 * NT) = kr2;
        *kslot(tid + 3 * NT) = kr3;
    };
    const float* vb = vcache + (size_t)g * max_t * HS;
    auto vaddr = [&](int c, int f) __attribute__((always_inline)) {
        return reinterpret_cast<const float4*>(vb + (size_t)min(c * kPqKeys + f / TPQ, nblk - 1) * HS + 4 * (f % TPQ));
    };
    auto vfetch = [&](int c) __attribute__((always_inline)) {
        vr0 = *vaddr(c, tid);
        vr1 = *vaddr(c, tid + NT);
        vr2 = *vaddr(c, tid + 2 * NT);
        vr3 = *vaddr(c, tid + 3 * NT);
    };
    kfetch(0);
    {   // the block's q rows (one float4 per thread)
        const float4 v = *reinterpret_cast<const float4*>(q + (size_t)min(qi, T - 1) * q_stride + (size_t)h * HS + 4 * quad);
        *reinterpret_cast<float4*>(qsm + ql * HSP + 4 * quad) = v;
    }
    vfetch(0);   // the first V chunk rides behind the scores
    // scores
    const int tl = tid % kPqKeys, qg = tid / kPqKeys;
    const float rs = sqrtf((float)HS);
    constexpr int NV = (HS & ~7) >> 2;   // float4 blocks added unfused, then the fused rest
    for (int c = 0; c < nchunks; c++) {
        __syncthreads();   // the previous chunk's dots are done (and, first, the q rows stored)
        kstore();
        __syncthreads();
        if (c + 1 < nchunks) kfetch(c + 1);
        const float4* k4 = reinterpret_cast<const float4*>(kvs + tl * HSP);
        const float4* qb = reinterpret_cast<const float4*>(qsm + qg * J * HSP);
        float sc[J];
#pragma unroll
        for (int j = 0; j < J; j++) sc[j] = 0.0f;
#pragma unroll 4
        for (int cc = 0; cc < NV; cc++) {
            const float4 kv = k4[cc];
            float4 qv[J];
#pragma unroll
            for (int j = 0; j < J; j++) qv[j] = qb[j * (HSP / 4) + cc];
#pragma unroll
            for (int j = 0; j < J; j++) {
                sc[j] = sc[j] + qv[j].x * kv.x;
                sc[j] = sc[j] + qv[j].y * kv.y;
                sc[j] = sc[j] + qv[j].z * kv.z;
                sc[j] = sc[j] + qv[j].w * kv.w;
            }
        }
#pragma unroll
        for (int cc = NV; cc < TPQ; cc++) {
            const float4 kv = k4[cc];
#pragma unroll
            for (int j = 0; j < J; j++) {
                const float4 qv = qb[j * (HSP / 4) + cc];
                sc[j] = __builtin_fmaf(qv.x, kv.x, sc[j]);
                sc[j] = __builtin_fmaf(qv.y, kv.y, sc[j]);
                sc[j] = __builtin_fmaf(qv.z, kv.z, sc[j]);
                sc[j] = __builtin_fmaf(qv.w, kv.w, sc[j]);
            }
        }
        const int t = c * kPqKeys + tl;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int qj = q0 + qg * J + j;
            if (qj < T && t <= pos0 + qj) ep[(qg * J + j) * kPqPitch + t] = sc[j] / rs;
        }
    }
    __syncthreads();
    // softmax (k_attn_softmax_b): max, exp, serial sum, divide
    constexpr int KMAX = kPqMaxKeys / TPQ;
    float sv[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; k++) sv[k] = e[min(quad + TPQ * k, max(n - 1, 0))];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < KMAX; k++)
        if (quad + TPQ * k < n) m = fmaxf(m, sv[k]);
    m = group_max<TPQ>(m);
#pragma unroll
    for (int k = 0; k < KMAX; k++)
        if (quad + TPQ * k < n) e[quad + TPQ * k] = exp_runq(sv[k] - m);
    __syncthreads();
    if (quad == 0 && n > 0) red[ql] = serial_sum(e, n);
    __syncthreads();
    const float sum = red[ql];
    for (int t = quad; t < n; t += TPQ) e[t] = e[t] / sum;
    // p*V (k_attn_pv_b's order)
    float4* vt = reinterpret_cast<float4*>(kvs);   // [kPqKeys][TPQ]
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int c = 0; c < nchunks; c++) {
        __syncthreads();   // the previous chunk's reads are done (and, first, the p rows written)
        vt[tid] = vr0;
        vt[tid + NT] = vr1;
        vt[tid + 2 * NT] = vr2;
        vt[tid + 3 * NT] = vr3;
        __syncthreads();
        if (c + 1 < nchunks) vfetch(c + 1);
        const int tn = min(kPqKeys, n - c * kPqKeys);
        const float* pr = e + c * kPqKeys;
        int t = 0;
        for (; t + 8 <= tn; t += 8) {
            float pv[8];
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                pv[k] = pr[t + k];
                v[k] = vt[(t + k) * TPQ + quad];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                acc.x = __builtin_fmaf(pv[k], v[k].x, acc.x);
                acc.y = __builtin_fmaf(pv[k], v[k].y, acc.y);
                acc.z = __builtin_fmaf(pv[k], v[k].z, acc.z);
                acc.w = __builtin_fmaf(pv[k], v[k].w, acc.w);
            }
        }
        for (; t < tn; t++) {
            const float pv = pr[t];
            const float4 v = vt[t * TPQ + quad];
            acc.x = __builtin_fmaf(pv, v.x, acc.x);
            acc.y = __builtin_fmaf(pv, v.y, acc.y);
            acc.z = __builtin_fmaf(pv, v.z, acc.z);
            acc.w = __builtin_fmaf(pv, v.w, acc.w);
        }
    }
    const bool in = qi < T;
    const int dim = n_heads * HS, e0 = h * HS + 4 * quad;    // first of this thread's four elements
    if (!pf.xqp) {
        if (in) *reinterpret_cast<float4*>(out + (size_t)qi * dim + e0) = acc;
        return;
    }
    // Q8 of the output (k_quantize): the G/4 threads of a group
    const float a0 = in ? acc.x : 0.0f, a1 = in ? acc.y : 0.0f, a2 = in ? acc.z : 0.0f, a3 = in ? acc.w : 0.0f;
    const float amax = fmaxf(fmaxf(fabsf(a0), fabsf(a1)), fmaxf(fabsf(a2), fabsf(a3)));
    const float s = q8_scale(group_max<G / 4>(amax));
    const float r = q8_recip(s);
    const int qa = q8_value_fast(a0, s, r), qb = q8_value_fast(a1, s, r), qc = q8_value_fast(a2, s, r),
              qd = q8_value_fast(a3, s, r);
    const int sum_q = group_isum<G / 4>(qa + qb + qc + qd);
    if (!in) return;
    constexpr int CH = G / 4;
    const int j0 = e0 % G;
    int8_t* dst = pf.xqp + (size_t)qi * dim + (e0 - j0);
    auto put = [&](int j, int qv) __attribute__((always_inline)) {
        const int jj = j % CH;
        dst[pf.bits == 4 ? j - jj + ((jj & 1) ? jj / 2 : CH / 2 + jj / 2) : j] = (int8_t)qv;
    };
    put(j0, qa);
    put(j0 + 1, qb);
    put(j0 + 2, qc);
    put(j0 + 3, qd);
    if (j0 == 0) pf.rec[(size_t)(e0 / G) * T + qi] = pf_record(s, sum_q, pf.bits);
}

// ---------------------------------------------------------------------------
// Single-query attention in the reference's exact order in ONE kernel
// (runq.c:367-391, softmax :307-318): the same operations as k_attn_scores
// + k_attn_softmax_v, bit for bit, without the second launch and the scores'
// round trip through memory.  Workgroup (head h, slice of kVDims output
// elements); its 8 waves
//   scores   one position per thread per round of kAfThreads positions:
//            the K row straight from the cache into registers (HS/4
//            float4), q broadcast from LDS, products rounded and added in
//            index order, / sqrtf(HS); scores kept in registers;
//   softmax  workgroup max, e_t = exp_runq(s_t - max), the sum of e_t in
//            position order (one lane, serial_sum), p_t = e_t / sum;
//   p*V      one lane per output element of the slice, fma(p_t, v_t[i],
//            acc) in position order (serial_pv) over chunks of kAfChunk
//            positions, transposed into LDS; the next chunk's loads are in
//            flight while the current one is folded.
// Every slice recomputes its head's scores (the K rows come from L2 after
// the first); the slices of a head are numbered so that they run on one
// XCD (workgroup id = slice * n_heads + h, ids dealt round-robin over 8
// XCDs) when n_heads is a multiple of 8.
constexpr int kAfThreads = 512;
constexpr int kAfChunk = 512;                                   // V positions per LDS chunk
constexpr int kAfStride = kAfChunk + 4;                         // LDS row of one element's chunk
constexpr int kAfVPer = kAfChunk * kVDims / 4 / kAfThreads;     // float4 per thread per chunk
constexpr int kAfRounds = kScorePer * kAttnThreads / kAfThreads;  // positions per thread (n <= 4096)
constexpr int kAfDefaultMax = kScorePer * kAttnThreads;         // see attention_fused_max
__host__ __device__ constexpr size_t attn_fused_lds_bytes(int max_t, int hs) {
    return ((size_t)(hs + 3) / 4 * 4 + (size_t)(max_t + 3) / 4 * 4 + kRingSlack + 2 * kVDims * kAfStride +
            kRingSlack + 16 + 64) * sizeof(float);
}
template <int HS, int KIL>
__global__ __launch_bounds__(kAfThreads) void k_attn_fused(
    const float* __restrict__ q, const float* __restrict__ kcache, const float* __restrict__ vcache,
    float* __restrict__ out, const int* __restrict__ meta, int pos_arg, int kv_mul, int n_heads, int max_t) {
#pragma clang fp contract(off)
    static_assert(HS % kVDims == 0 && HS % 8 == 0, "head size");
    constexpr int F4 = HS / 4;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* qs = smem;                                        // [HS]
    float* p = qs + (HS + 3) / 4 * 4;                        // [max_t] scores, e_t, then p_t
    float* vt = p + (max_t + 3) / 4 * 4 + kRingSlack;        // [2][kVDims][kAfStride]
    float* red = vt + 2 * kVDims * kAfStride + kRingSlack;   // [8] wave maxima, [8] sum
    uint64_t* etab = reinterpret_cast<uint64_t*>(red + 16);  // [32] exp table
    const int h = blockIdx.x % n_heads, d0 = (blockIdx.x / n_heads) * kVDims;
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE;
    const int n = meta_pos(meta, pos_arg) + 1;
    const float4* kbase = reinterpret_cast<const float4*>(kcache + (size_t)(h / kv_mul) * max_t * HS);
    const float* vbase = vcache + (size_t)(h / kv_mul) * max_t * HS + d0;
    const int nchunks = (n + kAfChunk - 1) / kAfChunk;

    // loads in the order they are needed (they complete in order): q and
    // the first round's K rows here, the first V chunk after the scores
    // (they share one HBM-bound stream, and V is not needed before the
    // softmax sum, so K arrives sooner).  The q load and its LDS store
    // are unconditional (clamped index; duplicates store equal values): a
    // load or store under a thread condition can be sunk behind the later
    // loads, and waiting for it then waits for them.  In the first round
    // and chunk (all of a short context), whole waves past the context skip
    // their K and V loads (wave-uniform branches), so that the per-CU load
    // path carries only positions that are used; the later ones load
    // clamped positions unconditionally, so that the next chunk's loads
    // stay in flight while the current one is folded.
    const float4 qv = reinterpret_cast<const float4*>(q + (size_t)h * HS)[min(tid, F4 - 1)];
    float4 kr[F4];
    auto load_k = [&](int t, bool skip) {   // column-interleaved: one coalesced KiB per column and wave
        if (skip && __builtin_amdgcn_readfirstlane(t) >= n) return;
        t = min(t, n - 1);
#pragma unroll
        for (int f = 0; f < F4; f++) kr[f] = KIL ? kbase[(size_t)f * max_t + t] : kbase[(size_t)t * F4 + f];
    };
    load_k(tid, true);
    float4 vr[kAfVPer];
    auto load_chunk = [&](int c, bool skip) {
#pragma unroll
        for (int k = 0; k < kAfVPer; k++) {
            const int e = tid + kAfThreads * k;                  // float4 index in the chunk
            const int r = e / (kVDims / 4), c4 = e % (kVDims / 4);
            const int t = c * kAfChunk + r;              // positions >= n are never folded
            if (skip && __builtin_amdgcn_readfirstlane(t) >= n) continue;
            vr[k] = *reinterpret_cast<const float4*>(vbase + (size_t)min(t, n - 1) * HS + 4 * c4);
        }
    };
    auto store_chunk = [&](int buf) {   // transposed: vt[buf][element][position]
        float* dst = vt + buf * kVDims * kAfStride;
#pragma unroll
        for (int k = 0; k < kAfVPer; k++) {
            const int e = tid + kAfThreads * k;
            const int r = e / (kVDims / 4), c4 = e % (kVDims / 4);
            dst[(4 * c4 + 0) * kAfStride + r] = vr[k].x;
            dst[(4 * c4 + 1) * kAfStride + r] = vr[k].y;
            dst[(4 * c4 + 2) * kAfStride + r] = vr[k].z;
            dst[(4 * c4 + 3) * kAfStride + r] = vr[k].w;
        }
    };
    // the exp table through the scalar cache (uniform loads: no vector
    // memory traffic, no 512 lanes per workgroup on one table)
    uint64_t tabv = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) tabv = (lane & 31) == i ? kExp2Tab[i] : tabv;
    reinterpret_cast<float4*>(qs)[min(tid, F4 - 1)] = qv;
    if (wv == 0) etab[lane & 31] = tabv;
    __syncthreads();   // qs, etab

    // scores: round r covers positions r*kAfThreads + tid
    float s[kAfRounds];
    float m = -INFINITY;
    const float4* q4 = reinterpret_cast<const float4*>(qs);
#pragma unroll
    for (int r = 0; r < kAfRounds; r++) {
        s[r] = -INFINITY;
        if (kAfThreads * r >= n) continue;   // uniform
        const int t = kAfThreads * r + tid;
        if (r > 0) load_k(t, false);
        float score = 0.0f;
#pragma unroll
        for (int f = 0; f < F4; f++) {
            const float4 qv = q4[f];
            score = score + qv.x * kr[f].x;
            score = score + qv.y * kr[f].y;
            score = score + qv.z * kr[f].z;
            score = score + qv.w * kr[f].w;
        }
        if (t < n) {
            s[r] = score / sqrtf((float)HS);
            m = fmaxf(m, s[r]);
        }
    }
    load_chunk(0, true);   // V after K: the scores need only K
    m = group_max<L2Q_WAVE>(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kAfThreads / L2Q_WAVE; w++) m = fmaxf(m, red[w]);
    float e[kAfRounds];
#pragma unroll
    for (int r = 0; r < kAfRounds; r++) {
        const int t = kAfThreads * r + tid;
        e[r] = 0.0f;
        if (kAfThreads * r < n && t < n) {
            e[r] = exp_runq_t(s[r] - m, etab);
            p[t] = e[r];
        }
    }
    __syncthreads();
    if (tid == 0) red[8] = serial_sum(p, n);
    __syncthreads();
    const float sum = red[8];
#pragma unroll
    for (int r = 0; r < kAfRounds; r++) {
        const int t = kAfThreads * r + tid;
        if (kAfThreads * r < n && t < n) p[t] = e[r] / sum;
    }
    store_chunk(0);
    __syncthreads();

    float acc = 0.0f;
    for (int c = 0; c < nchunks; c++) {
        if (c + 1 < nchunks) load_chunk(c + 1, false);
        if (wv == 0 && lane < kVDims) {
            const int tb = c * kAfChunk;
            acc = serial_pv(p + tb, vt + (c & 1) * kVDims * kAfStride + lane * kAfStride, min(kAfChunk, n - tb), acc);
        }
        if (c + 1 < nchunks) store_chunk((c + 1) & 1);
        __syncthreads();
    }
    if (wv == 0 && lane < kVDims) out[(size_t)h * HS + d0 + lane] = acc;
}

// ---------------------------------------------------------------------------
// int8 KV cache (v5-cuda-fused/run.cu:41-48, INT8_KV): k8 / v8 laid out
// [n_kv][max_t][hs] int8 with one fp32 scale per (kv head, position),
// ks / vs [n_kv][max_t].

// Row `pos` of kv head blockIdx.x, k (blockIdx.y == 0, rotated first when a
// RoPE table is given) or v: amax, s = amax/127 (1e-8 when 0), q =
// clamp(rint(v/s), -127, 127) with the IEEE quotient
// (v5-cuda-fused/run.cu:204-249).  One wave; element pairs (2p, 2p+1) on
// lane p mod 64.
constexpr int kKv8Pairs = kAttnMaxHs / 2 / L2Q_WAVE;   // pairs per lane (hs <= 256)
// One wave quantizes one row: src[0..hs) (rotated first when a RoPE table
// is given) -> int8 row `dst` (global, may be null) and, with TO_LDS,
// `ldst` (LDS), scale to *scale / *lscale (lane 0).  (TO_LDS is a template
// argument: a run-time null test of a generic pointer that holds an LDS
// address miscompiles on gfx950 in some kernels.)
template <bool TO_LDS>
__device__ __forceinline__ void kv8_quant_row(const float* __restrict__ src, const float* __restrict__ rope, int pos,
                                              int hs, int lane, int8_t* dst, float* scale, int8_t* ldst,
                                              float* lscale) {
    float2 val[kKv8Pairs];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kKv8Pairs; i++) {
        const int p = lane + L2Q_WAVE * i;
        val[i] = make_float2(0.0f, 0.0f);
        if (2 * p < hs) {
            float2 x = reinterpret_cast<const float2*>(src)[p];
            if (rope) {   // the fp32 path's rotation (RoPE table of the position)
                const float c = rope[(size_t)pos * hs + 2 * p], s = rope[(size_t)pos * hs + 2 * p + 1];
                x = make_float2(__builtin_fmaf(x.x, c, -(x.y * s)), __builtin_fmaf(x.x, s, x.y * c));
            }
            val[i] = x;
            amax = fmaxf(amax, fmaxf(fabsf(x.x), fabsf(x.y)));
        }
    }
    amax = group_max<L2Q_WAVE>(amax);
    float sc = amax / 127.0f;
    if (sc == 0.0f) sc = 1e-8f;
#pragma unroll
    for (int i = 0; i < kKv8Pairs; i++) {
        const int p = lane + L2Q_WAVE * i;
        if (2 * p < hs) {
            const int q0 = q8_value(val[i].x, sc), q1 = q8_value(val[i].y, sc);
            const uint16_t w = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
            if (dst) *reinterpret_cast<uint16_t*>(dst + 2 * p) = w;
            if constexpr (TO_LDS) *reinterpret_cast<uint16_t*>(ldst + 2 * p) = w;
        }
    }
    if (lane == 0) {
        if (scale) *scale = sc;
        if constexpr (TO_LDS) *lscale = sc;
    }
}

__global__ __launch_bounds__(L2Q_WAVE) void k_kv8_append(
    const float* __restrict__ k, const float* __restrict__ v, int8_t* __restrict__ k8, int8_t* __restrict__ v8,
    float* __restrict__ ks, float* __restrict__ vs, const float* __restrict__ rope, const int* __restrict__ meta,
    int pos_arg, int hs, int max_t, int src_rows) {
    // row blockIdx.z of k / v ([n_kv][src_rows][hs]; a decode step: one row)
    // to cache position pos + blockIdx.z
    const int g = blockIdx.x, isv = blockIdx.y, lane = threadIdx.x;
    const int pos = meta_pos(meta, pos_arg) + blockIdx.z;
    const size_t row = (size_t)g * max_t + pos;
    const size_t src = ((size_t)g * src_rows + blockIdx.z) * hs;
    kv8_quant_row<false>((isv ? v : k) + src, isv ? nullptr : rope, pos, hs, lane, (isv ? v8 : k8) + row * hs,
                  (isv ? vs : ks) + row, nullptr, nullptr);
}

// Attention over the int8 cache (v5-cuda-fused/run.cu:350-410), one kernel
// per step, a workgroup of kA8Threads threads per head:
//   append   when kst / vst (the rotated k row and the v row of the step,
//            [n_kv][hs] staging) are given: waves 0 and 1 quantize the
//            head's kv row (kv8_quant_row, as k_kv8_append) into LDS; the
//            group's first head also writes it to the cache (the others
//            compute the same bits for their own use, so no workgroup waits
//            for another);
//   scores   (run.cu:362-371) score_t = (q . k8_t) / sqrt(hs) * ks_t, all
//            threads, kA8Threads/4 positions per round with the next
//            round's K in flight, four lanes per position, each summing the
//            4-element chunks c = 4*sub + 16*i with FMAs, then a two-step
//            butterfly; into LDS (position pos from the LDS row when
//            appending);
//   softmax  (run.cu:373-398) max as a block reduction; the sum: thread j
//            sums positions j, j + 1024, ...; then the wave butterfly, then a
//            pairwise tree over the 16 waves ((w0 + w1) + (w2 + w3)) + ...;
//            e_t * vs_t kept in LDS;
//   p*V      thread (slice, g) accumulates elements 4g..4g+3 over positions
//            t = slice (mod slices), 1024/(hs/4) slices; the slices are
//            added in LDS in slice order and divided by the sum.
// Every reduction has a fixed order (restated by the oracle's
// orc_attention_kv8_ordered), so results are reproducible bit for bit.
// Needs hs % 16 == 0.
constexpr int kA8Threads = 1024;
constexpr int kA8Waves = kA8Threads / L2Q_WAVE;
constexpr int kA8Chunks = kAttnMaxHs / 16;               // K dwords per lane and position (hs <= 256)
// Byte b of w as a signed value.
__device__ __forceinline__ float sbyte(int w, int b) { return (float)((w << (24 - 8 * b)) >> 24); }
__host__ __device__ constexpr size_t attn8_fused_lds_bytes(int max_t) {
    return ((size_t)(max_t + 3) / 4 * 4 + 4 * kA8Threads + 3 * kA8Waves + 2 * kAttnMaxHs / 4 + 64) * sizeof(float);
}
__global__ __launch_bounds__(kA8Threads) void k_attn8_fused(
    const float* __restrict__ q, const float* __restrict__ kst, const float* __restrict__ vst,
    int8_t* __restrict__ k8, int8_t* __restrict__ v8, float* __restrict__ ks, float* __restrict__ vs,
    float* __restrict__ out, const int* __restrict__ meta, int pos_arg, int kv_mul, int hs, int max_t,
    int q_stride, int out_stride) {
    extern __shared__ __attribute__((aligned(16))) float smf[];
    float* sc = smf;                                   // [max_t] scores, then e_t * vs_t
    float* part = sc + (max_t + 3) / 4 * 4;            // [slices][hs] partial sums
    float* red = part + 4 * kA8Threads;                // [16] wave maxima, [16] wave sums, [2] row scales
    int8_t* krow = reinterpret_cast<int8_t*>(red + 3 * kA8Waves);   // [hs] appended k row, then [hs] v row
    int8_t* vrow = krow + kAttnMaxHs;
    uint64_t* etab = reinterpret_cast<uint64_t*>(vrow + kAttnMaxHs);   // [32] exp table
    const int h = blockIdx.x, hk = h / kv_mul;
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE, sub = tid & 3;
    // query blockIdx.y of a batch (prefill): position pos + blockIdx.y, its q
    // row and output row at the given strides (a decode step: one query)
    const int pos = meta_pos(meta, pos_arg) + blockIdx.y;
    q += (size_t)blockIdx.y * q_stride;
    out += (size_t)blockIdx.y * out_stride;
    const int n = pos + 1;
    const bool append = kst != nullptr;
    const size_t prow = (size_t)hk * max_t + pos;
    if (append && wv < 2) {
        const bool first = h % kv_mul == 0;
        if (wv == 0)
            kv8_quant_row<true>(kst + (size_t)hk * hs, nullptr, pos, hs, lane, first ? k8 + prow * hs : nullptr,
                          first ? ks + prow : nullptr, krow, red + 2 * kA8Waves);
        else
            kv8_quant_row<true>(vst + (size_t)hk * hs, nullptr, pos, hs, lane, first ? v8 + prow * hs : nullptr,
                          first ? vs + prow : nullptr, vrow, red + 2 * kA8Waves + 1);
    }

    // scores: the lane's q chunks in registers, the next round's K dwords
    // loaded before the current round's FMAs
    const float rs = sqrtf((float)hs);
    const int nch = hs / 16;
    const float* qh = q + (size_t)h * hs;
    float4 qr[kA8Chunks];
#pragma unroll
    for (int i = 0; i < kA8Chunks; i++)
        qr[i] = i < nch ? *reinterpret_cast<const float4*>(qh + 4 * sub + 16 * i) : make_float4(0, 0, 0, 0);
    const int8_t* kb = k8 + (size_t)hk * max_t * hs;
    int kw[kA8Chunks];
    auto load_round = [&](int t0, int (&w)[kA8Chunks]) {
        const int tc = min(t0 + tid / 4, n - 1);
#pragma unroll
        for (int i = 0; i < kA8Chunks; i++)
            if (i < nch) w[i] = *reinterpret_cast<const int*>(kb + (size_t)tc * hs + 4 * sub + 16 * i);
    };
    load_round(0, kw);
    if (wv == 2) {   // the exp table through the scalar cache (uniform loads)
        uint64_t tabv = 0;
#pragma unroll
        for (int i = 0; i < 32; i++) tabv = (lane & 31) == i ? kExp2Tab[i] : tabv;
        etab[lane & 31] = tabv;
    }
    __syncthreads();   // the appended row and the exp table in LDS
    for (int t0 = 0; t0 < n; t0 += kA8Threads / 4) {
        int kn[kA8Chunks];
        load_round(min(t0 + kA8Threads / 4, n - 1), kn);
        const int t = t0 + tid / 4;
        const bool own = append && min(t, n - 1) == pos;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kA8Chunks; i++) {
            if (i < nch) {
                const int w = own ? *reinterpret_cast<const int*>(krow + 4 * sub + 16 * i) : kw[i];
                acc = __builtin_fmaf(qr[i].x, sbyte(w, 0), acc);
                acc = __builtin_fmaf(qr[i].y, sbyte(w, 1), acc);
                acc = __builtin_fmaf(qr[i].z, sbyte(w, 2), acc);
                acc = __builtin_fmaf(qr[i].w, sbyte(w, 3), acc);
            }
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        if (sub == 0 && t < n) sc[t] = acc / rs * (own ? red[2 * kA8Waves] : ks[(size_t)hk * max_t + t]);
#pragma unroll
        for (int i = 0; i < kA8Chunks; i++) kw[i] = kn[i];
    }
    __syncthreads();

    // softmax
    float m = -INFINITY;
    for (int t = tid; t < n; t += kA8Threads) m = fmaxf(m, sc[t]);
    m = group_max<L2Q_WAVE>(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kA8Threads / L2Q_WAVE; w++) m = fmaxf(m, red[w]);
    {
        float sum = 0.0f;
        for (int t = tid; t < n; t += kA8Threads) {
            const float e = exp_runq_t(sc[t] - m, etab);   // the host C library's expf, bit for bit
            sum += e;
            sc[t] = e * (append && t == pos ? red[2 * kA8Waves + 1] : vs[(size_t)hk * max_t + t]);
        }
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (lane == 0) red[kA8Waves + wv] = sum;
    }
    __syncthreads();
    float tree[kA8Waves];
#pragma unroll
    for (int w = 0; w < kA8Waves; w++) tree[w] = red[kA8Waves + w];
#pragma unroll
    for (int width = kA8Waves / 2; width >= 1; width /= 2)
#pragma unroll
        for (int w = 0; w < width; w++) tree[w] = tree[2 * w] + tree[2 * w + 1];
    const float sum = tree[0];
    const int groups = hs / 4, slices = kA8Threads / groups;
    const int gi = tid % groups, slice = tid / groups;
    if (slice < slices) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const int8_t* vb = v8 + (size_t)hk * max_t * hs + 4 * gi;
#pragma unroll 8
        for (int t = slice; t < n; t += slices) {
            const int w = append && t == pos ? *reinterpret_cast<const int*>(vrow + 4 * gi)
                                             : *reinterpret_cast<const int*>(vb + (size_t)t * hs);
            const float p = sc[t];
            acc.x = __builtin_fmaf(p, sbyte(w, 0), acc.x);
            acc.y = __builtin_fmaf(p, sbyte(w, 1), acc.y);
            acc.z = __builtin_fmaf(p, sbyte(w, 2), acc.z);
            acc.w = __builtin_fmaf(p, sbyte(w, 3), acc.w);
        }
        *reinterpret_cast<float4*>(part + (size_t)slice * hs + 4 * gi) = acc;
    }
    __syncthreads();
    for (int d = tid; d < hs; d += kA8Threads) {
        float s2 = 0.0f;
        for (int sl = 0; sl < slices; sl++) s2 += part[(size_t)sl * hs + d];
        out[(size_t)h * hs + d] = s2 / sum;
    }
}

// ---------------------------------------------------------------------------
// int8-KV attention split over the context (the int8-KV engine's decode
// attention and l2q_attention_kv8_ex with L2Q_ATTN_SPLIT_CONTEXT): the
// v5-cuda-fused/run.cu:350-410 formula with the cache read by n_heads x S
// workgroups instead of one per head.  Workgroup (head h, split s) of 256
// threads covers positions [s*C, min((s+1)*C, n)), C = ceil(n/S) <= 256;
// its float order is restated by the oracle's orc_attention_kv8_split:
//   append   the split holding pos quantizes the step's staged k and v rows
//            into LDS (waves 0 and 1, kv8_quant_row); the kv group's first
//            head also writes them to the cache;
//   scores   k_attn8_fused's per-position order (four lanes per position,
//            chain `sub` over the chunks 4*sub + 16*i with FMAs, butterfly
//            (a0+a1)+(a2+a3), then / sqrtf(hs) * ks_t), 64 positions per
//            round with the next round's K in flight;
//   softmax  m_s = the split's max; e_t = expf(s_t - m_s) (exp_runq_t);
//            l_s = thread j's e_{t0+j}, wave butterflies, (w0+w1)+(w2+w3);
//   p*V      256/(hs/4) slices x hs/4 element groups: fma(e_t*vs_t, v8_t,
//            acc) over t = t0 + slice, + slices, ...; slices added in order;
//   merge    as k_attn_flash: wave 0 stores (m_s, l_s, o_s) with agent-scope
//            stores, waits for them, arrives on the head's counter; the S-th
//            arrival merges in split order: w_s = expf(m_s - M),
//            L = sum w_s*l_s, out = (sum fma(w_s, o_s)) / L, and resets the
//            counter.  No workgroup waits on another.
constexpr int kA8sThreads = 256;
constexpr int kA8sMaxC = 256;
__host__ __device__ constexpr size_t attn8_split_lds_bytes(int S, int hs) {
    return ((size_t)kA8sMaxC + 4 * kA8sThreads + 16 + 2 * kAttnMaxHs / 4 + 64 + (size_t)S * (hs + 2)) * sizeof(float);
}
__global__ __launch_bounds__(kA8sThreads) void k_attn8_split(
    const float* __restrict__ q, const float* __restrict__ kst, const float* __restrict__ vst,
    int8_t* __restrict__ k8, int8_t* __restrict__ v8, float* __restrict__ ks, float* __restrict__ vs,
    float* __restrict__ out, float* __restrict__ part, unsigned* __restrict__ cnt, const int* __restrict__ meta,
    int pos_arg, int kv_mul, int hs, int max_t, int q_stride, int out_stride) {
    extern __shared__ __attribute__((aligned(16))) float smf[];
    float* sc = smf;                                   // [C] scores, then e_t * vs_t
    float* psl = sc + kA8sMaxC;                        // [slices][hs] p*V partials, then the partial
    float* red = psl + 4 * kA8sThreads;                // [4] wave maxima, [4] wave sums, [2] row scales
    int8_t* krow = reinterpret_cast<int8_t*>(red + 16);   // [hs] appended k row, then [hs] v row
    int8_t* vrow = krow + kAttnMaxHs;
    uint64_t* etab = reinterpret_cast<uint64_t*>(vrow + kAttnMaxHs);   // [32] exp table
    float* mrg = reinterpret_cast<float*>(etab + 32);  // [S][hs + 2] merge staging
    __shared__ int is_last;
    const int h = blockIdx.x, s = blockIdx.y, S = gridDim.y, hk = h / kv_mul;
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE, sub = tid & 3;
    // query blockIdx.z of a batch (prefill): position pos + blockIdx.z, its
    // q / output rows at the given strides, its own partials and counters
    // (a decode step: one query)
    const int pos = meta_pos(meta, pos_arg) + blockIdx.z;
    q += (size_t)blockIdx.z * q_stride;
    out += (size_t)blockIdx.z * out_stride;
    part += (size_t)blockIdx.z * gridDim.x * S * (hs + 2);
    cnt += (size_t)blockIdx.z * gridDim.x;
    const int n = pos + 1;
    const int C = (n + S - 1) / S;
    const int t0 = min(s * C, n), t1 = min(n, t0 + C), mn = t1 - t0;
    const bool append = kst != nullptr && t0 <= pos && pos < t1;
    const size_t prow = (size_t)hk * max_t + pos;
    if (append && wv < 2) {   // wave 0 the k row, wave 1 the v row (one call with per-wave arguments)
        const bool first = h % kv_mul == 0;
        const float* src = (wv == 0 ? kst : vst) + (size_t)hk * hs;
        int8_t* cache = wv == 0 ? k8 : v8;
        float* scale = wv == 0 ? ks : vs;
        kv8_quant_row<true>(src, nullptr, pos, hs, lane, first ? cache + prow * hs : nullptr, first ? scale + prow : nullptr,
                      wv == 0 ? krow : vrow, red + 8 + wv);
    }
    const float rs = sqrtf((float)hs);
    const int nch = hs / 16;
    const float* qh = q + (size_t)h * hs;
    float4 qr[kA8Chunks];
#pragma unroll
    for (int i = 0; i < kA8Chunks; i++)
        qr[i] = i < nch ? *reinterpret_cast<const float4*>(qh + 4 * sub + 16 * i) : make_float4(0, 0, 0, 0);
    const int8_t* kb = k8 + (size_t)hk * max_t * hs;
    const int tl = max(t1 - 1, 0);
    int kw[kA8Chunks];
    auto load_round = [&](int r0, int (&w)[kA8Chunks]) {
        const int tc = min(t0 + r0 + tid / 4, tl);
#pragma unroll
        for (int i = 0; i < kA8Chunks; i++)
            if (i < nch) w[i] = *reinterpret_cast<const int*>(kb + (size_t)tc * hs + 4 * sub + 16 * i);
    };
    if (mn > 0) load_round(0, kw);
    if (wv == 2) {   // the exp table through the scalar cache (uniform loads)
        uint64_t tabv = 0;
#pragma unroll
        for (int i = 0; i < 32; i++) tabv = (lane & 31) == i ? kExp2Tab[i] : tabv;
        etab[lane & 31] = tabv;
    }
    __syncthreads();   // the appended rows and the exp table in LDS
    for (int r0 = 0; r0 < mn; r0 += kA8sThreads / 4) {
        int kn[kA8Chunks];
        load_round(min(r0 + kA8sThreads / 4, mn - 1), kn);
        const int t = t0 + r0 + tid / 4;
        const bool own = append && min(t, tl) == pos;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kA8Chunks; i++) {
            if (i < nch) {
                const int w = own ? *reinterpret_cast<const int*>(krow + 4 * sub + 16 * i) : kw[i];
                acc = __builtin_fmaf(qr[i].x, sbyte(w, 0), acc);
                acc = __builtin_fmaf(qr[i].y, sbyte(w, 1), acc);
                acc = __builtin_fmaf(qr[i].z, sbyte(w, 2), acc);
                acc = __builtin_fmaf(qr[i].w, sbyte(w, 3), acc);
            }
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        // both scales read, the value selected (a select of the two addresses
        // would become one generic load, which the compiler mishandles here)
        const float kso = red[8], ksc = ks[(size_t)hk * max_t + min(t, tl)];
        if (sub == 0 && t < t1) sc[t - t0] = acc / rs * (own ? kso : ksc);
#pragma unroll
        for (int i = 0; i < kA8Chunks; i++) kw[i] = kn[i];
    }
    __syncthreads();
    // the split's softmax
    float m = tid < mn ? sc[tid] : -INFINITY;
    m = group_max<L2Q_WAVE>(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
    if (tid < mn) {
        const int t = t0 + tid;
        const float e = exp_runq_t(sc[tid] - m, etab);   // the host C library's expf, bit for bit
        l = l + e;
        const float vso = red[9], vsc = vs[(size_t)hk * max_t + t];
        sc[tid] = e * (append && t == pos ? vso : vsc);
    }
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
    if (lane == 0) red[4 + wv] = l;
    __syncthreads();
    l = (red[4] + red[5]) + (red[6] + red[7]);
    // p*V slices
    const int groups = hs / 4, slices = kA8sThreads / groups;
    const int gi = tid % groups, sl = tid / groups;
    if (sl < slices) {
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const int8_t* vb = v8 + (size_t)hk * max_t * hs + 4 * gi;
        for (int j = sl; j < mn; j += slices) {
            const int t = t0 + j;
            const int wo = *reinterpret_cast<const int*>(vrow + 4 * gi);
            const int wc = *reinterpret_cast<const int*>(vb + (size_t)t * hs);
            const int w = append && t == pos ? wo : wc;
            const float p = sc[j];
            acc.x = __builtin_fmaf(p, sbyte(w, 0), acc.x);
            acc.y = __builtin_fmaf(p, sbyte(w, 1), acc.y);
            acc.z = __builtin_fmaf(p, sbyte(w, 2), acc.z);
            acc.w = __builtin_fmaf(p, sbyte(w, 3), acc.w);
        }
        *reinterpret_cast<float4*>(psl + (size_t)sl * hs + 4 * gi) = acc;
    }
    __syncthreads();
    float od[kAttnMaxHs / L2Q_WAVE];   // this lane's partial elements d = lane + 64k (wave 0)
    if (wv == 0) {
#pragma unroll
        for (int k = 0; k < kAttnMaxHs / L2Q_WAVE; k++) {
            const int d = lane + L2Q_WAVE * k;
            float o = 0.0f;
            if (d < hs)
                for (int k2 = 0; k2 < slices; k2++) o = o + psl[(size_t)k2 * hs + d];
            od[k] = o;
        }
    }
    // the partial (wave 0, agent-scope stores), then the arrival
    float* pp = part + ((size_t)h * S + s) * (hs + 2);
    auto put = [](float* a, float v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto get = [](const float* a) {
        return __hip_atomic_load(const_cast<float*>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (wv == 0) {
#pragma unroll
        for (int k = 0; k < kAttnMaxHs / L2Q_WAVE; k++)
            if (lane + L2Q_WAVE * k < hs) put(pp + lane + L2Q_WAVE * k, od[k]);
        if (lane == 0) {
            put(pp + hs, mn > 0 ? m : -INFINITY);
            put(pp + hs + 1, mn > 0 ? l : 0.0f);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's partial stores are acknowledged
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0)
            is_last = __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (unsigned)(S - 1);
    }
    __syncthreads();
    if (!is_last) return;
    // merge in split order
    const float* ph = part + (size_t)h * S * (hs + 2);
    const int total = S * (hs + 2);
    for (int e0 = 0; e0 < total; e0 += 8 * kA8sThreads) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int e = e0 + k * kA8sThreads + tid;
            v[k] = e < total ? get(ph + e) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int e = e0 + k * kA8sThreads + tid;
            if (e < total) mrg[e] = v[k];
        }
    }
    __syncthreads();
    float M = -INFINITY;
    for (int k = 0; k < S; k++) M = fmaxf(M, mrg[k * (hs + 2) + hs]);
    float* wsp = psl;   // [S] merge weights w_s (the p*V partials are no longer needed)
    if (tid < S) {
        const float ms = mrg[tid * (hs + 2) + hs];
        wsp[tid] = ms == -INFINITY ? 0.0f : exp_runq_t(ms - M, etab);
    }
    __syncthreads();
    float L = 0.0f;
    for (int k = 0; k < S; k++) L = L + wsp[k] * mrg[k * (hs + 2) + hs + 1];
    for (int d = tid; d < hs; d += kA8sThreads) {
        float acc = 0.0f;
        for (int k = 0; k < S; k++) acc = __builtin_fmaf(wsp[k], mrg[k * (hs + 2) + d], acc);
        out[(size_t)h * hs + d] = acc / L;
    }
    if (tid == 0) __hip_atomic_store(cnt + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge the S partials of each head: out = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s.
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part_o,
                                                      const float* __restrict__ part_ml,
                                                      float* __restrict__ out, int S, int hs) {
    const int h = blockIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < S; s++) M = fmaxf(M, part_ml[((size_t)h * S + s) * 2]);
    float L = 0.0f;
    for (int s = 0; s < S; s++) {
        const float ms = part_ml[((size_t)h * S + s) * 2];
        if (ms != -INFINITY) L += expf(ms - M) * part_ml[((size_t)h * S + s) * 2 + 1];
    }
    for (int d = threadIdx.x; d < hs; d += blockDim.x) {
        float acc = 0.0f;
        for (int s = 0; s < S; s++) {
            const float ms = part_ml[((size_t)h * S + s) * 2];
            if (ms != -INFINITY) acc += expf(ms - M) * part_o[((size_t)h * S + s) * hs + d];
        }
        out[(size_t)h * hs + d] = acc / L;
    }
}

// ---------------------------------------------------------------------------
// Split-context single-query attention in ONE kernel (the engine's
// tolerance mode; runq.c:367-391 + softmax :307-318 up to rounding).
// Workgroup (head h, split s) of kFlThreads threads covers positions
// [s*C, min((s+1)*C, n)), C = ceil(n/S) <= kFlMaxC, n = pos + 1:
//   scores  blocks of 64 positions: wave w forms the dot over chunks
//           [w*HS/16, (w+1)*HS/16) of q.k for position lane (two FMA chains),
//           the four wave partials are added in LDS ((p0 + p1) + (p2 + p3))
//           and scaled by 1/sqrtf(HS); K in either cache layout (k_index);
//   softmax m = max s_t, e_t = expf(s_t - m), l = sum e_t (wave sums, then
//           (l0 + l1) + (l2 + l3));
//   p*V     thread (row slice r of 8, float4 column c) accumulates e_t v_t
//           over t = r, r + 8, ...; the 8 slices are added in order;
//   merge   the partial (m, l, o[HS]) goes to part[h][s] through agent-scope
//           stores; once they are acknowledged the workgroup arrives on the
//           head's counter (agent-scope atomic), and the one whose arrival
//           is the S-th reads the head's S partials with agent-scope loads,
//           merges them in split order, out = sum_s w_s o_s / sum_s w_s l_s
//           with w_s = expf(m_s - M), and resets the counter for the next
//           launch.  (Release / acquire fences would write back and
//           invalidate the whole L2 once per workgroup: measured 2x slower.)
// Every workgroup arrives exactly once (empty splits too), and no
// workgroup waits on another, so the kernel always drains.
constexpr int kFlThreads = 256;
constexpr int kFlBlock = 64;     // positions per score block (one per lane)
constexpr int kFlMaxC = 256;     // positions per workgroup
constexpr int kFlSlices = kFlThreads / 32;
constexpr int kFlMaxSplits = 64;
template <int HS, int KIL>
__global__ __launch_bounds__(kFlThreads) void k_attn_flash(
    const float* __restrict__ q, const float* __restrict__ kcache, const float* __restrict__ vcache,
    float* __restrict__ out, float* __restrict__ part, unsigned* __restrict__ cnt, const int* __restrict__ meta,
    int pos_arg, int kv_mul, int max_t) {
    static_assert(HS == 48 || HS == 64 || HS == 128, "head size");
    constexpr int F4 = HS / 4;           // float4 chunks per row
    constexpr int CW = F4 / 4;           // chunks per wave in the scores
    constexpr int NV = kFlBlock / kFlSlices;   // V rows per thread per block
    __shared__ float4 qs[F4];
    __shared__ float sp[4][kFlBlock];
    __shared__ float sc[kFlMaxC];
    __shared__ float4 po[kFlSlices][32];
    __shared__ float red[8];
    __shared__ float wsm[2 * kFlMaxSplits];   // merge: w_s, then w_s * l_s
    __shared__ float mrg[kFlMaxSplits * (HS + 2)];   // merge: the head's partials
    __shared__ int is_last;
    const int h = blockIdx.x, s = blockIdx.y, S = gridDim.y;
    const int tid = threadIdx.x, lane = tid & (L2Q_WAVE - 1), wv = tid / L2Q_WAVE;
    const int n = meta_pos(meta, pos_arg) + 1;
    const int C = (n + S - 1) / S;
    const int t0 = min(s * C, n), t1 = min(n, t0 + C);
    const int m_n = t1 - t0;
    const int kvh = h / kv_mul;
    const float4* k4 = reinterpret_cast<const float4*>(kcache);
    const float4* v4 = reinterpret_cast<const float4*>(vcache) + (size_t)kvh * max_t * F4;
    auto kaddr = [&](int t, int c) {
        return KIL ? k4 + ((size_t)(kvh * F4 + c) * max_t + t) : k4 + ((size_t)kvh * max_t + t) * F4 + c;
    };
    const int r = tid >> 5, c4 = tid & 31;   // p*V: row slice, float4 column (c4 < F4 active)
    const int tl = max(t1 - 1, 0);           // clamped positions load a valid row, never used

    // loads in the order they are needed: q, the first block's K, its V
    if (tid < F4) qs[tid] = reinterpret_cast<const float4*>(q + (size_t)h * HS)[tid];
    float4 kr[CW], vr[NV];
    auto load_k = [&](int b) {
        const int t = min(t0 + kFlBlock * b + lane, tl);
#pragma unroll
        for (int c = 0; c < CW; c++) kr[c] = *kaddr(t, wv * CW + c);
    };
    auto load_v = [&](int b) {
#pragma unroll
        for (int k = 0; k < NV; k++)
            vr[k] = c4 < F4 ? v4[(size_t)min(t0 + kFlBlock * b + r + kFlSlices * k, tl) * F4 + c4]
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    const int nblk = (m_n + kFlBlock - 1) / kFlBlock;
    if (nblk > 0) {
        load_k(0);
        load_v(0);
    }
    __syncthreads();   // qs
    const float rs = sqrtf((float)HS);
    for (int b = 0; b < nblk; b++) {
        if (b > 0) load_k(b);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int c = 0; c < CW; c++) {
            const float4 qv = qs[wv * CW + c];
            a0 = __builtin_fmaf(qv.x, kr[c].x, a0);
            a1 = __builtin_fmaf(qv.y, kr[c].y, a1);
            a0 = __builtin_fmaf(qv.z, kr[c].z, a0);
            a1 = __builtin_fmaf(qv.w, kr[c].w, a1);
        }
        sp[wv][lane] = a0 + a1;
        __syncthreads();
        if (tid < kFlBlock) {
            const int j = kFlBlock * b + tid;
            if (j < m_n) sc[j] = ((sp[0][tid] + sp[1][tid]) + (sp[2][tid] + sp[3][tid])) / rs;
        }
        __syncthreads();
    }
    float m = -INFINITY;
    for (int j = tid; j < m_n; j += kFlThreads) m = fmaxf(m, sc[j]);
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
    for (int j = tid; j < m_n; j += kFlThreads) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        l += e;
    }
    l = wave_sum(l);
    if (lane == 0) red[4 + wv] = l;
    __syncthreads();   // sc holds e_t; red[4..8) the wave sums
    l = (red[4] + red[5]) + (red[6] + red[7]);
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int b = 0; b < nblk; b++) {
        if (b > 0) load_v(b);
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int j = kFlBlock * b + r + kFlSlices * k;
            if (j < m_n) {
                const float e = sc[j];
                o.x = __builtin_fmaf(e, vr[k].x, o.x);
                o.y = __builtin_fmaf(e, vr[k].y, o.y);
                o.z = __builtin_fmaf(e, vr[k].z, o.z);
                o.w = __builtin_fmaf(e, vr[k].w, o.w);
            }
        }
    }
    po[r][c4] = o;
    __syncthreads();
    // the partial, written by wave 0 with agent-scope stores (written
    // through to the device-coherent level, no L2 writeback of the whole
    // cache as a release fence would do); once they are acknowledged, the
    // arrival on the head's counter
    float* pp = part + ((size_t)h * S + s) * (HS + 2);
    auto put = [](float* a, float v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto get = [](const float* a) {
        return __hip_atomic_load(const_cast<float*>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (tid < F4) {
        float4 acc = po[0][tid];
#pragma unroll
        for (int k = 1; k < kFlSlices; k++) {
            const float4 x = po[k][tid];
            acc.x += x.x; acc.y += x.y; acc.z += x.z; acc.w += x.w;
        }
        put(pp + 4 * tid, acc.x);
        put(pp + 4 * tid + 1, acc.y);
        put(pp + 4 * tid + 2, acc.z);
        put(pp + 4 * tid + 3, acc.w);
    }
    if (tid == 0) {
        put(pp + HS, m_n > 0 ? m : -INFINITY);
        put(pp + HS + 1, m_n > 0 ? l : 0.0f);
    }
    if (wv == 0) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's partial stores are acknowledged
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (tid == 0)
            is_last = __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (unsigned)(S - 1);
    }
    __syncthreads();
    if (!is_last) return;
    // merge the head's S partials in split order: staged into LDS by
    // batches of independent agent-scope loads (the other workgroups'
    // partials, read past every non-coherent cache level)
    const float* ph = part + (size_t)h * S * (HS + 2);
    const int total = S * (HS + 2);
    for (int e0 = 0; e0 < total; e0 += 8 * kFlThreads) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int e = e0 + k * kFlThreads + tid;
            v[k] = e < total ? get(ph + e) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int e = e0 + k * kFlThreads + tid;
            if (e < total) mrg[e] = v[k];
        }
    }
    __syncthreads();
    float M = -INFINITY;
    for (int k = 0; k < S; k++) M = fmaxf(M, mrg[k * (HS + 2) + HS]);
    if (tid < S) {
        const float ms = mrg[tid * (HS + 2) + HS];
        const float w = ms == -INFINITY ? 0.0f : expf(ms - M);
        wsm[tid] = w;
        wsm[kFlMaxSplits + tid] = w * mrg[tid * (HS + 2) + HS + 1];
    }
    __syncthreads();
    if (tid < HS) {
        float L = 0.0f, acc = 0.0f;
        for (int k = 0; k < S; k++) {
            L += wsm[kFlMaxSplits + k];
            acc = __builtin_fmaf(wsm[k], mrg[k * (HS + 2) + tid], acc);
        }
        out[(size_t)h * HS + tid] = acc / L;
    }
    if (tid == 0) __hip_atomic_store(cnt + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Greedy argmax (runq.c:578-585: first index of the maximum).  One
// workgroup; each thread takes float4 chunks t, t + 1024, ... (v 16-byte
// aligned), the loads of eight chunks in flight at once, and scans its
// elements in ascending index order, so its first maximum is kept; the
// reduction prefers the smaller index on equal values.
constexpr int kArgmaxThreads = 1024;
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax(const float* __restrict__ v, int n, int* __restrict__ out) {
    __shared__ float bv[kArgmaxThreads / L2Q_WAVE];
    __shared__ int bi[kArgmaxThreads / L2Q_WAVE];
    // the reference starts from v[0] and takes v[i] > max: NaNs are never
    // taken, and a NaN at index 0 makes the answer 0 (every comparison with
    // it is false); v[0] is read with the first loads, not at the end
    const float v0 = v[0];
    float best = -INFINITY;
    int idx = n;   // sentinel larger than every index
    const int n4 = n / 4;
    const float4* v4 = reinterpret_cast<const float4*>(v);
    for (int base = 0; base < n4; base += 8 * kArgmaxThreads) {
        float4 x[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int f = base + (int)threadIdx.x + kArgmaxThreads * k;
            x[k] = v4[min(f, n4 - 1)];
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int f = base + (int)threadIdx.x + kArgmaxThreads * k;
            if (f < n4) {
                if (x[k].x > best) { best = x[k].x; idx = 4 * f; }
                if (x[k].y > best) { best = x[k].y; idx = 4 * f + 1; }
                if (x[k].z > best) { best = x[k].z; idx = 4 * f + 2; }
                if (x[k].w > best) { best = x[k].w; idx = 4 * f + 3; }
            }
        }
    }
    for (int i = 4 * n4 + (int)threadIdx.x; i < n; i += kArgmaxThreads) {
        const float x = v[i];
        if (x > best) { best = x; idx = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, L2Q_WAVE);
        const int oi = __shfl_xor(idx, o, L2Q_WAVE);
        if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
    }
    const int w = threadIdx.x / L2Q_WAVE;
    if ((threadIdx.x & (L2Q_WAVE - 1)) == 0) { bv[w] = best; bi[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int ix = bi[0];
        for (int k = 1; k < (int)(blockDim.x / L2Q_WAVE); k++)
            if (bv[k] > b || (bv[k] == b && bi[k] < ix)) { b = bv[k]; ix = bi[k]; }
        out[0] = ix < n && !isnan(v0) ? ix : 0;
    }
}

// Embedding row gather (runq.c:332-333) for the diagnostic path.
__global__ void k_embed(const float* __restrict__ emb, const int* __restrict__ meta, float* __restrict__ x,
                        int dim) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < dim) x[i] = emb[(size_t)meta[0] * dim + i];
}

// Elementwise exp_runq (exposed for the exhaustive identity check).
__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = exp_runq(x[i]);
}

// One-time un-bias of QLL8 weights (u8 = q + 128 -> s8), 16 bytes a thread.
__global__ void k_unbias(const uint8_t* __restrict__ src, int8_t* __restrict__ dst, size_t n) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
    if (i + 16 <= n) {
        uint4 u = *reinterpret_cast<const uint4*>(src + i);
        u.x ^= 0x80808080u; u.y ^= 0x80808080u; u.z ^= 0x80808080u; u.w ^= 0x80808080u;
        *reinterpret_cast<uint4*>(dst + i) = u;
    } else {
        for (size_t j = i; j < n; j++) dst[j] = (int8_t)(src[j] ^ 0x80u);
    }
}

}  // namespace l2q
