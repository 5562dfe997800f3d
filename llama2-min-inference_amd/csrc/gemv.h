// gemv.h - batch-1 GEMV over group-quantized INT8 / packed-INT4 weights.
//
// out[r] = sum_b ws[r,b] * (xs[b] * d_u8(r,b) - xt[b])  (runq.c:142-159)
// with d(r,b) = sum_{j<G} w[r,bG+j] * xq[bG+j] the exact int32 group dot.
//
// Mapping (wave64, no MFMA: at batch 1 this is a pure weight stream):
//   - one wave owns R consecutive rows;
//   - lane j owns groups j, j+64, j+128, ... (T of them) of every row, so
//     each lane streams whole groups (16/32/64 bytes) with 128-bit loads
//     and a wave reads 64 consecutive groups of a row in one sweep;
//   - the lane's activation groups (int8 + scale + bias term) are loaded
//     once into registers and reused for all R rows;
//   - INT4 nibbles are consumed in place (see dot8_q4_x16): no unpack to
//     bytes, two v_dot4_i32_i8 per 8 weights;
//   - all R*T weight loads are issued before the first dot product so a
//     wave keeps R*T*G/2 (INT4) bytes in flight;
//   - per-(row, group) terms are folded in group order by one lane per row,
//     reproducing the reference's float accumulation bit for bit.
#pragma once
#include "device.h"

namespace l2q {

struct GemvArgs {
    float* out;
    const int8_t* xq;
    const float* xs;
    const void* w;
    const float* ws;
    int rows;
    int cols;
    int32_t* dots;   // optional [rows][cols/G] int32 group dots
};

template <int BITS, int G>
struct GroupShape {
    static constexpr int GB = G * BITS / 8;   // weight bytes per group
    static constexpr int NV = GB / 16;        // 128-bit loads per group
    static constexpr int AW = G / 4;          // activation dwords per group
    static_assert(GB % 16 == 0, "group must be a multiple of 16 bytes");
};

// Activations of the groups a lane owns, held in registers.
template <int BITS, int G, int T>
struct LaneActs {
    int x[T][G / 4];    // INT8: natural order; INT4: [even dwords | odd dwords]
    float xs[T];
    float xt[T];
    int sq[T];
};

template <int BITS, int G, int T>
__device__ __forceinline__ void load_lane_acts(LaneActs<BITS, G, T>& A, const int8_t* __restrict__ xq,
                                               const float* __restrict__ xs, int nb, int lane) {
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int g = lane + L2Q_WAVE * t;
        int raw[G / 4];
        if (g < nb) {
            const uint4* p = reinterpret_cast<const uint4*>(xq + (size_t)g * G);
#pragma unroll
            for (int v = 0; v < G / 16; v++) {
                uint4 u = p[v];
                raw[4 * v + 0] = (int)u.x; raw[4 * v + 1] = (int)u.y;
                raw[4 * v + 2] = (int)u.z; raw[4 * v + 3] = (int)u.w;
            }
            A.xs[t] = xs[g];
        } else {
#pragma unroll
            for (int k = 0; k < G / 4; k++) raw[k] = 0;
            A.xs[t] = 0.0f;
        }
        int s = 0;
#pragma unroll
        for (int k = 0; k < G / 4; k++) s = dot4(raw[k], 0x01010101, s);
        A.sq[t] = s;
        A.xt[t] = q8_bias_term(A.xs[t], s);
        if (BITS == 4) {
#pragma unroll
            for (int k = 0; k < G / 8; k++) {
                A.x[t][k] = even_bytes(raw[2 * k], raw[2 * k + 1]);
                A.x[t][G / 8 + k] = odd_bytes(raw[2 * k], raw[2 * k + 1]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < G / 4; k++) A.x[t][k] = raw[k];
        }
    }
}

// Exact int32 dot of one group given its NV 128-bit weight words.
template <int BITS, int G, int T>
__device__ __forceinline__ int group_dot(const uint4* wv, const LaneActs<BITS, G, T>& A, int t) {
    constexpr int NV = GroupShape<BITS, G>::NV;
    int d = 0;
    if (BITS == 8) {
#pragma unroll
        for (int v = 0; v < NV; v++) {
            d = dot4((int)wv[v].x, A.x[t][4 * v + 0], d);
            d = dot4((int)wv[v].y, A.x[t][4 * v + 1], d);
            d = dot4((int)wv[v].z, A.x[t][4 * v + 2], d);
            d = dot4((int)wv[v].w, A.x[t][4 * v + 3], d);
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; v++) {
            d = dot8_q4_x16(wv[v].x, A.x[t][4 * v + 0], A.x[t][G / 8 + 4 * v + 0], d);
            d = dot8_q4_x16(wv[v].y, A.x[t][4 * v + 1], A.x[t][G / 8 + 4 * v + 1], d);
            d = dot8_q4_x16(wv[v].z, A.x[t][4 * v + 2], A.x[t][G / 8 + 4 * v + 2], d);
            d = dot8_q4_x16(wv[v].w, A.x[t][4 * v + 3], A.x[t][G / 8 + 4 * v + 3], d);
        }
        d >>= 4;   // exact: the x16 dot is a multiple of 16
    }
    return d;
}

constexpr int kGemvRowsPerWave = 4;
constexpr int kGemvWaves = 4;
constexpr int kGemvRowsPerBlock = kGemvRowsPerWave * kGemvWaves;

// LDS bytes of k_gemv for a given group count (per wave: ws and term of
// 4 rows, rows padded to nb+1 floats so the folding lanes hit distinct banks).
__host__ __device__ constexpr size_t gemv_lds_bytes(int nb) {
    return (size_t)kGemvWaves * kGemvRowsPerWave * (nb + 1) * 2 * sizeof(float);
}

// GEMV on pre-quantized activations.  Each wave owns 4 rows; after the
// dot products every (row, group) term t_b = xs_b*d_u8 - xt_b and its weight
// scale ws_b go to LDS, and one lane per row folds them in group order,
// sum = fma(ws_b, t_b, sum) for b = 0, 1, ..., exactly the sequence of
// roundings of the reference loop (runq.c:150-156), so the fp32 output is
// bit-identical to it.  Grid: ceil(rows/16) workgroups of 256 threads.
template <int BITS, int G, int T>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    constexpr int NV = GroupShape<BITS, G>::NV;
    constexpr int GB = GroupShape<BITS, G>::GB;
    constexpr int R = kGemvRowsPerWave;
    extern __shared__ float lds[];
    const int lane = threadIdx.x & (L2Q_WAVE - 1);
    const int wv = threadIdx.x / L2Q_WAVE;
    const int row0 = blockIdx.x * kGemvRowsPerBlock + wv * R;
    if (row0 >= a.rows) return;   // whole wave idle (wave-uniform)
    const int nb = a.cols / G;
    const int stride = nb + 1;
    float* ws_l = lds + (size_t)wv * R * stride * 2;
    float* t_l = ws_l + R * stride;
    const size_t rowbytes = (size_t)a.cols * BITS / 8;
    const uint8_t* wbase = static_cast<const uint8_t*>(a.w);

    // Activations first (L2-resident, short latency), then every weight
    // load of this wave, so the activation set-up overlaps the weight stream.
    LaneActs<BITS, G, T> A;
    load_lane_acts<BITS, G, T>(A, a.xq, a.xs, nb, lane);

    uint4 wv4[R][T][NV];
    float wsc[R][T];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int g = lane + L2Q_WAVE * t;
            if (row < a.rows && g < nb) {
                const uint8_t* p = wbase + (size_t)row * rowbytes + (size_t)g * GB;
#pragma unroll
                for (int v = 0; v < NV; v++) wv4[r][t][v] = load_stream(p + 16 * v);
                wsc[r][t] = a.ws[(size_t)row * nb + g];
            } else {
#pragma unroll
                for (int v = 0; v < NV; v++) wv4[r][t][v] = make_uint4(0, 0, 0, 0);
                wsc[r][t] = 0.0f;
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int g = lane + L2Q_WAVE * t;
            const int d = group_dot<BITS, G, T>(wv4[r][t], A, t);
            if (g < nb) {
                if (a.dots && row < a.rows) a.dots[(size_t)row * nb + g] = d;
                ws_l[r * stride + g] = wsc[r][t];
                t_l[r * stride + g] = group_term(A.xs[t], A.xt[t], d, A.sq[t]);
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < R && row0 + lane < a.rows) {
        const float* wp = ws_l + lane * stride;
        const float* tp = t_l + lane * stride;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) sum = __builtin_fmaf(wp[b], tp[b], sum);
        a.out[row0 + lane] = sum;
    }
}

}  // namespace l2q
