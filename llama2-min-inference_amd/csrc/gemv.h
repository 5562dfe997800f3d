// gemv.h - batch-1 GEMV over group-quantized INT8 / packed-INT4 weights,
// with the prologues and epilogues of the decode step fused in.
//
// out[r] = sum_b ws[r,b] * (xs[b] * d_u8(r,b) - xt[b])  (runq.c:142-159)
// with d(r,b) = sum_{j<G} w[r,bG+j] * xq[bG+j] the exact int32 group dot,
// d_u8 = d + 128*sum(xq_b) and xt[b] = xs[b]*128*sum(xq_b).
//
// Mapping (wave64, no MFMA: at batch 1 this is a pure weight stream):
//   - a workgroup (4 waves) owns tiles of 4*R consecutive rows, a wave R;
//   - a row is read in sweeps of 1 KiB: in sweep s lane j loads the 16
//     bytes at s*1024 + 16*j, so every load instruction of a wave covers
//     one contiguous KiB (the best-coalesced form of the stream);
//   - a group spans P = G*BITS/128 consecutive lanes (1, 2 or 4); their
//     partial int32 dots and activation sums are combined with lane
//     shuffles, exactly (integer adds);
//   - the activation chunk a lane needs is the same for every row, so it is
//     loaded (or taken from the prologue's LDS copy) once into registers;
//   - every weight load of the wave is issued before any dependent work, so
//     the activation set-up and the prologue run while weights stream in;
//   - INT4 nibbles are consumed in place (see dot8_q4_x16): no unpack to
//     bytes, two v_dot4_i32_i8 per 8 weights;
//   - per-(row, group) terms go to LDS and one lane per row folds them in
//     group order, sum = fma(ws_b, t_b, sum), reproducing the reference's
//     float accumulation bit for bit.
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
};


constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * L2Q_WAVE;
constexpr int kSweepBytes = 16 * L2Q_WAVE;   // one 128-bit load per lane

// Rows per wave: 4, or 2 for long rows (keeps the weight registers of a
// tile within the register file).
__host__ __device__ constexpr int gemv_rows_per_wave(int NS) { return NS <= 4 ? 4 : 2; }
__host__ __device__ constexpr int gemv_rows_per_block(int NS) { return kGemvWaves * gemv_rows_per_wave(NS); }
__host__ __device__ constexpr int gemv_sweeps(int bits, int cols) { return (cols * bits / 8 + kSweepBytes - 1) / kSweepBytes; }

// A prologue thread holds ceil(cols/1024) float4 chunks of the input; with
// cols*BITS/8 <= 1024*NS that is at most NS*8/BITS.
__host__ __device__ constexpr int prologue_chunks(int NS, int BITS) { return NS * 8 / BITS; }

// LDS layout (floats): [fold: 4 waves x R rows x (nb+1) x 2][act: cols int8 + nb scales][vs: cols (kNorm)][misc 4]
__host__ __device__ constexpr size_t gemv_fold_floats(int nb, int NS) {
    return (size_t)gemv_rows_per_block(NS) * (nb + 1) * 2;
}
__host__ __device__ constexpr size_t gemv_lds_bytes(int pro, int cols, int group, int bits) {
    return (gemv_fold_floats(cols / group, gemv_sweeps(bits, cols)) + (pro == kPreq ? 0 : (size_t)cols / 4 + cols / group) +
            (pro == kNorm ? (size_t)cols : 0) + 4) * sizeof(float);
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

// Activation chunks of a lane, held in registers for all rows.
template <int BITS, int G, int NS>
struct LaneActs {
    int x[NS][32 / BITS];     // INT8: natural order; INT4: [even dwords | odd dwords] per 8 elements
    float xs[NS];                    // scale of the chunk's group
    float xt[NS];                    // bias term of the group (runq.c:137)
    int sq[NS];                      // sum(q) over the whole group
};

// Raw activation words of lane chunk (s, lane): loads only.
template <int BITS, int G, int NS>
__device__ __forceinline__ void load_lane_raw(int (&raw)[NS][32 / BITS], float (&sc)[NS], const int8_t* xq,
                                              const float* xs, int cols, int lane) {
    using C = Chunk<BITS, G>;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int e0 = (s * kSweepBytes + 16 * lane) * 8 / BITS;   // first element of the chunk
        if (e0 < cols) {
            const uint4* p = reinterpret_cast<const uint4*>(xq + e0);
#pragma unroll
            for (int v = 0; v < C::AD / 4; v++) {
                const uint4 u = p[v];
                raw[s][4 * v + 0] = (int)u.x; raw[s][4 * v + 1] = (int)u.y;
                raw[s][4 * v + 2] = (int)u.z; raw[s][4 * v + 3] = (int)u.w;
            }
            sc[s] = xs[e0 / G];
        } else {
#pragma unroll
            for (int k = 0; k < C::AD; k++) raw[s][k] = 0;
            sc[s] = 0.0f;
        }
    }
}

// Sum over the P lanes of a group (P = 1, 2, 4): exact integer adds.
template <int P>
__device__ __forceinline__ int group_lanes_isum(int v) {
    if (P >= 2) v += __shfl_xor(v, 1, L2Q_WAVE);
    if (P >= 4) v += __shfl_xor(v, 2, L2Q_WAVE);
    return v;
}

// sum(q) over the group, the bias term and (INT4) the even/odd byte split.
template <int BITS, int G, int NS>
__device__ __forceinline__ void finish_lane_acts(LaneActs<BITS, G, NS>& A, const int (&raw)[NS][32 / BITS],
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

// Partial int32 dot of one 16-byte weight chunk (x16 for INT4).
template <int BITS, int G, int NS>
__device__ __forceinline__ int chunk_dot(const uint4 w, const LaneActs<BITS, G, NS>& A, int s) {
    using C = Chunk<BITS, G>;
    if (BITS == 8) {
        int d = dot4((int)w.x, A.x[s][0], 0);
        d = dot4((int)w.y, A.x[s][1], d);
        d = dot4((int)w.z, A.x[s][2], d);
        return dot4((int)w.w, A.x[s][3], d);
    } else {
        int d = dot8_q4_x16(w.x, A.x[s][0], A.x[s][C::AD / 2 + 0], 0);
        d = dot8_q4_x16(w.y, A.x[s][1], A.x[s][C::AD / 2 + 1], d);
        d = dot8_q4_x16(w.z, A.x[s][2], A.x[s][C::AD / 2 + 2], d);
        return dot8_q4_x16(w.w, A.x[s][3], A.x[s][C::AD / 2 + 3], d);
    }
}

// Sum of squares of v[0..n) in the reference's order (runq.c:295-302):
// lanes 0..15 of the calling wave each run one of its 16 FMA accumulators
// (j = l, l+16, ...), then the _mm512_reduce_add_ps tree, then the tail as
// GCC compiles the scalar loop (a block of 8 unfused, then FMAs).  The
// result is valid in lane 0.  v is in LDS; all 64 lanes must call.
__device__ __forceinline__ float runq_sumsq(const float* v, int n, int lane) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (lane < 16) {
        const int nfull = n & ~15;
        int j = 0;
        for (; j + 16 * 16 <= nfull; j += 16 * 16) {
            float a[16];
#pragma unroll
            for (int u = 0; u < 16; u++) a[u] = v[j + 16 * u + lane];
#pragma unroll
            for (int u = 0; u < 16; u++) acc = __builtin_fmaf(a[u], a[u], acc);
        }
        for (; j < nfull; j += 16) {
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

// Workgroup prologue: quantize (for kNorm: residual add + RMSNorm first) the
// fp32 vector into LDS act_q[cols] / act_s[nb].  Thread t handles float4
// chunks c = t + 256*k (elements 4c..4c+3); a group is G/4 consecutive
// threads of one wave, so group maxima are lane-group reductions.  The
// inputs were loaded to registers by the caller before the weight loads.
template <int G, int PRO, int PC, int RC>
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
            const int c = tid + kGemvThreads * k;
            if (c < nchunks) {
                float4 v = xin[k];
                if (a.resid) { v.x += res[k].x; v.y += res[k].y; v.z += res[k].z; v.w += res[k].w; }
                xin[k] = v;
                *reinterpret_cast<float4*>(vs + 4 * c) = v;
                if (a.x_out && blockIdx.x == 0) *reinterpret_cast<float4*>(a.x_out + 4 * c) = v;
            }
        }
        __syncthreads();
        if (tid < L2Q_WAVE) {
            const float ss = runq_sumsq(vs, n, lane);
            if (lane == 0) misc[0] = 1.0f / sqrtf(ss / (float)n + 1e-5f);
        }
        __syncthreads();
        inv = misc[0];
    }
#pragma unroll
    for (int k = 0; k < kProChunks; k++) {
        if (kGemvThreads * k >= nchunks) break;   // uniform across the workgroup
        const int c = tid + kGemvThreads * k;
        const bool in = c < nchunks;
        float4 o = xin[k];
        if constexpr (PRO == kNorm) {
            o.x = nw[k].x * (inv * o.x); o.y = nw[k].y * (inv * o.y);
            o.z = nw[k].z * (inv * o.z); o.w = nw[k].w * (inv * o.w);
        }
        if (!in) o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float m = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
        m = group_max<G / 4>(m);
        const float s = q8_scale(m);
        if (in) {
            const int q0 = q8_value(o.x, s), q1 = q8_value(o.y, s), q2 = q8_value(o.z, s), q3 = q8_value(o.w, s);
            const int packed = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((q3 & 0xff) << 24);
            reinterpret_cast<int*>(act_q)[c] = packed;
            if ((c % (G / 4)) == 0) act_s[c / (G / 4)] = s;
        }
    }
    __syncthreads();
}

// Persistent over row tiles: workgroup b handles tiles b, b + gridDim.x, ...
// (4*R rows each); the prologue runs once per workgroup and the next tile's
// weight loads are issued before the current tile's fold and epilogue.
template <int BITS, int G, int NS, int PRO, int EPI>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(GemvArgs a) {
    using C = Chunk<BITS, G>;
    constexpr int R = gemv_rows_per_wave(NS);
    constexpr int RB = gemv_rows_per_block(NS);
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int lane = threadIdx.x & (L2Q_WAVE - 1);
    const int wv = threadIdx.x / L2Q_WAVE;
    const int nb = a.cols / G;
    const int stride = nb + 1;
    const int ntiles = (a.rows + RB - 1) / RB;
    float* ws_l = lds + (size_t)wv * R * stride * 2;
    float* t_l = ws_l + R * stride;
    int8_t* act_q = reinterpret_cast<int8_t*>(lds + gemv_fold_floats(nb, NS));
    float* act_s = reinterpret_cast<float*>(act_q + a.cols);
    float* vs = act_s + nb;
    float* misc = vs + (PRO == kNorm ? a.cols : 0);
    const size_t rowbytes = (size_t)a.cols * BITS / 8;
    const uint8_t* wbase = static_cast<const uint8_t*>(a.w);
    const bool leader = (lane % C::P) == 0;

    // 1. prologue inputs first, so that waiting for them never waits on the
    //    weight loads issued after them (vector loads complete in order)
    constexpr int kProChunks = PRO == kPreq ? 1 : prologue_chunks(NS, BITS);
    constexpr int kResChunks = PRO == kNorm ? kProChunks : 1;
    float4 xin[kProChunks], res[kResChunks], nw[kResChunks];
    const int nchunks = a.cols / 4;
    if (PRO != kPreq) {
        const float* src = (PRO == kNorm && a.emb) ? a.emb + (size_t)a.meta[0] * a.cols : a.x_in;
#pragma unroll
        for (int k = 0; k < kProChunks; k++) {
            const int c = threadIdx.x + kGemvThreads * k;
            if (kGemvThreads * k < nchunks && c < nchunks) {
                xin[k] = reinterpret_cast<const float4*>(src)[c];
                if constexpr (PRO == kNorm) {
                    res[k] = a.resid ? reinterpret_cast<const float4*>(a.resid)[c] : make_float4(0, 0, 0, 0);
                    nw[k] = reinterpret_cast<const float4*>(a.norm_w)[c];
                }
            }
        }
    }
    int raw[NS][32 / BITS];
    float sc[NS];
    if (PRO == kPreq) load_lane_raw<BITS, G, NS>(raw, sc, a.xq, a.xs, a.cols, lane);
    __builtin_amdgcn_sched_barrier(0);

    // 2. weight loads of this wave's rows of a tile: chunk (r, s) is the 16
    //    bytes at row*rowbytes + s*1024 + 16*lane; the scale is loaded by
    //    the group's leader lane
    uint4 w4[R][NS];
    float wsc[R][NS];
    auto load_tile = [&](int tile) {
        const int row0 = tile * RB + wv * R;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const int off = s * kSweepBytes + 16 * lane;
                if (row < a.rows && off < (int)rowbytes) {
                    w4[r][s] = load_stream(wbase + (size_t)row * rowbytes + off);
                    wsc[r][s] = leader ? a.ws[(size_t)row * nb + off / C::GB] : 0.0f;
                } else {
                    w4[r][s] = make_uint4(0, 0, 0, 0);
                    wsc[r][s] = 0.0f;
                }
            }
        }
    };
    int tile = blockIdx.x;
    load_tile(tile);
    __builtin_amdgcn_sched_barrier(0);

    // 3. prologue (workgroup-wide) while the weights stream in
    if (PRO != kPreq) {
        prologue_compute<G, PRO, kProChunks, kResChunks>(a, xin, res, nw, act_q, act_s, vs, misc, nchunks);
        load_lane_raw<BITS, G, NS>(raw, sc, act_q, act_s, a.cols, lane);
    }
    LaneActs<BITS, G, NS> A;
    finish_lane_acts<BITS, G, NS>(A, raw, sc);

    for (; tile < ntiles; tile += gridDim.x) {
        const int row0 = tile * RB + wv * R;
        const bool active = row0 < a.rows;   // wave-uniform
        // 4. dots and per-group terms of this tile
        if (active) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = row0 + r;
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    const int off = s * kSweepBytes + 16 * lane;
                    int d = group_lanes_isum<C::P>(chunk_dot<BITS, G, NS>(w4[r][s], A, s));
                    if (BITS == 4) d >>= 4;   // exact: the x16 dot is a multiple of 16
                    if (leader && off < (int)rowbytes) {
                        const int g = off / C::GB;
                        if (a.dots && row < a.rows) a.dots[(size_t)row * nb + g] = d;
                        ws_l[r * stride + g] = wsc[r][s];
                        t_l[r * stride + g] = group_term(A.xs[s], A.xt[s], d, A.sq[s]);
                    }
                }
            }
        }
        // the next tile's weights stream in during this tile's fold
        if (tile + (int)gridDim.x < ntiles) load_tile(tile + gridDim.x);
        if (!active) continue;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // 5. ordered fold: lane r folds row row0 + r
        float sum = 0.0f;
        if (lane < R) {
            const float* wp = ws_l + lane * stride;
            const float* tp = t_l + lane * stride;
            for (int b = 0; b < nb; b++) sum = __builtin_fmaf(wp[b], tp[b], sum);
        }

        // 6. epilogue on lanes 0..R-1 (R is even: pairs stay in one wave)
        const int row = row0 + lane;
        if (EPI == kStore) {
            if (lane < R && row < a.rows) a.out[row] = sum;
        } else if (EPI == kRopeKV) {
            // rows come in (even, odd) pairs held by lanes (0,1), (2,3)
            const float other = __shfl_xor(sum, 1, L2Q_WAVE);
            if (lane < R && row < a.rows) {
                const int pos = a.meta[1];
                const bool odd = row & 1;
                const float v0 = odd ? other : sum, v1 = odd ? sum : other;
                if (row < a.dim + a.kv_dim) {            // q or k: rotate
                    const int e = row < a.dim ? row : row - a.dim;
                    const int hd = (e & ~1) % a.hs;
                    const float c = a.rope[(size_t)pos * a.hs + hd];
                    const float s = a.rope[(size_t)pos * a.hs + hd + 1];
                    const float r = odd ? __builtin_fmaf(v0, s, v1 * c) : __builtin_fmaf(v0, c, -(v1 * s));
                    if (row < a.dim) a.out[row] = r;
                    else a.kcache[((size_t)(e / a.hs) * a.max_t + pos) * a.hs + (e % a.hs)] = r;
                } else {                                  // v: appended as is
                    const int e = row - a.dim - a.kv_dim;
                    a.vcache[((size_t)(e / a.hs) * a.max_t + pos) * a.hs + (e % a.hs)] = sum;
                }
            }
        } else {   // kSwiglu: (w1, w3) pairs on lanes (0,1), (2,3)
            const float h3 = __shfl_xor(sum, 1, L2Q_WAVE);
            if (lane < R && (lane & 1) == 0 && row < a.rows) {
#pragma clang fp contract(off)
                float h = sum;
                h *= (1.0f / (1.0f + exp_runq(-h)));
                a.out[row >> 1] = h * h3;
            }
        }
        // the LDS fold area is reused by the next tile: keep the next
        // tile's term writes behind this tile's fold reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace l2q
