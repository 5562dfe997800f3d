// device.h - gfx950 device helpers shared by the decode kernels.
//
// Wave64 reductions, the Q8 group quantizer (runq.c:117-139 semantics, in
// registers), int8/int4 group dot products on v_dot4_i32_i8, and the
// per-group accumulation formula of runq.c:150-156.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define L2Q_WAVE 64

namespace l2q {

// Launch-shape limits shared by the kernels and their host launchers.
constexpr int kNormThreads = 1024;   // fused RMSNorm: one workgroup
constexpr int kNormMaxPer = 8;       // elements per thread -> n <= 8192
constexpr int kAttnThreads = 256;    // attention workgroup
constexpr int kAttnMaxHs = 256;      // largest head size

// Row pitch of the batched attention's score / probability rows [T][heads]
// [pitch]: max_t rounded up to 4, so the p rows read as float4 stay aligned
// for every cache length.
__host__ __device__ constexpr int attn_b_pitch(int max_t) { return (max_t + 3) / 4 * 4; }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 128-bit weight load.
#ifndef L2Q_INPUT_FIRST
#define L2Q_INPUT_FIRST 1
#endif
#ifndef L2Q_WEIGHT_NT
#define L2Q_WEIGHT_NT 1
#endif
__device__ __forceinline__ uint4 load_stream(const void* p) {
#if L2Q_WEIGHT_NT
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#else
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
#endif
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------------------
// Wave64 reductions (xor butterflies: every lane ends with the result).

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, L2Q_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, L2Q_WAVE));
    return v;
}

// Lane permutations inside 16-lane rows via DPP (a VALU operand modifier:
// no LDS round trip, unlike __shfl_*).  quad_perm [1,0,3,2] and [2,3,0,1]
// are lane^1 and lane^2; row_half_mirror maps lane i to 7-i within each
// 8-lane half row; row_mirror maps i to 15-i within the row.
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppMirror = 0x140, kDppHalfMirror = 0x141 };

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

// The values of lanes l and l ^ 16 (l ^ 32), in some order, without an
// LDS round trip: v_permlane16_swap / v_permlane32_swap (gfx950) of v with
// itself leave {v[l], v[l ^ 16]} in the two results of every lane (checked
// on the GPU), so a commutative reduction of the pair is the xor-16 (xor-32)
// butterfly step.
__device__ __forceinline__ void xor16_pair(unsigned v, unsigned& a, unsigned& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void xor32_pair(unsigned v, unsigned& a, unsigned& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}

// Max / integer sum over aligned groups of `W` consecutive lanes (W a power
// of two <= 64): every lane gets the result of its own group.  Both are
// exact in any order; within a 16-lane row the butterfly is xor1, xor2,
// half mirror, mirror (after the last two steps every lane has seen all 16),
// across rows the permlane swaps.
// group_max on unsigned values (the bit patterns of non-negative floats
// order as the floats do): one integer max per step, with the lane move
// folded into it.
template <int W>
__device__ __forceinline__ unsigned group_umax(unsigned v) {
    if (W >= 2) v = max(v, (unsigned)dpp_i<kDppXor1>((int)v));
    if (W >= 4) v = max(v, (unsigned)dpp_i<kDppXor2>((int)v));
    if (W >= 8) v = max(v, (unsigned)dpp_i<kDppHalfMirror>((int)v));
    if (W >= 16) v = max(v, (unsigned)dpp_i<kDppMirror>((int)v));
    unsigned a, b;
    if (W >= 32) { xor16_pair(v, a, b); v = max(a, b); }
    if (W >= 64) { xor32_pair(v, a, b); v = max(a, b); }
    return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
    if (W >= 2) v = fmaxf(v, dpp_f<kDppXor1>(v));
    if (W >= 4) v = fmaxf(v, dpp_f<kDppXor2>(v));
    if (W >= 8) v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    if (W >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
    unsigned a, b;
    if (W >= 32) { xor16_pair(__float_as_uint(v), a, b); v = fmaxf(__uint_as_float(a), __uint_as_float(b)); }
    if (W >= 64) { xor32_pair(__float_as_uint(v), a, b); v = fmaxf(__uint_as_float(a), __uint_as_float(b)); }
    return v;
}

template <int W>
__device__ __forceinline__ int group_isum(int v) {
    if (W >= 2) v += dpp_i<kDppXor1>(v);
    if (W >= 4) v += dpp_i<kDppXor2>(v);
    if (W >= 8) v += dpp_i<kDppHalfMirror>(v);
    if (W >= 16) v += dpp_i<kDppMirror>(v);
    unsigned a, b;
    if (W >= 32) { xor16_pair((unsigned)v, a, b); v = (int)(a + b); }
    if (W >= 64) { xor32_pair((unsigned)v, a, b); v = (int)(a + b); }
    return v;
}

// ---------------------------------------------------------------------------
// Q8 activation quantization of one value given its group's amax:
// s = amax/127 (1e-8 if 0), q = clamp(rint(x/s), +-127).  Division is the
// correctly rounded IEEE one (HIP default; never built with fast-math) and
// rintf is round-half-even, as lrintf in the reference.

// amax / 127 as the correctly rounded quotient of the reference, by one
// product and one FMA correction: s0 = amax * RN(1/127), then
// s = fma(fma(-s0, 127, amax), RN(1/127), s0), equal to the IEEE quotient for
// every finite amax >= 0 (fp32 denormals kept, as these kernels run; the
// identity is checked exhaustively by the CPU test suite).  Three
// instructions instead of the division sequence.
__device__ __forceinline__ float q8_scale(float amax) {
    constexpr float kInv127 = 1.0f / 127.0f;
    const float s0 = amax * kInv127;
    const float s = __builtin_fmaf(__builtin_fmaf(-s0, 127.0f, amax), kInv127, s0);
    return s == 0.0f ? 1e-8f : s;
}

__device__ __forceinline__ int q8_value(float x, float s) {
    float r = rintf(x / s);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

// q8_value_fast as the bits of rint(q) + 1.5*2^23: adding 1.5*2^23 rounds y
// (|y| < 128) to an integer, to nearest even as rintf does, and leaves that
// integer in the low bits, so the int8 value is the low byte of the result
// (no conversion instruction); the off-path quotient is clamped to +-127 and
// rounded the same way.
__device__ __forceinline__ unsigned q8_byte_fast(float x, float s, float r) {
    constexpr float kMagic = 0x1.8p23f;
    const float y = x * r;
    float t = y + kMagic;
    if (__builtin_expect(!(fabsf(y - (t - kMagic)) < 0.5f - 0x1p-13f), 0))
        t = fminf(fmaxf(x / s, -127.0f), 127.0f) + kMagic;
    return __float_as_uint(t);
}

// q8_value(x, s) without a division on the common path.  With r = rcp(s)
// (v_rcp_f32, within 1 ulp) y = x*r is within 4 ulp(y) of x/s, so rint(y)
// equals rint(fl(x/s)) unless y lies within that distance of a half-integer
// (the only places where the two can round differently), i.e. unless
// |y - rint(y)| >= 0.5 - margin; there, and for non-finite y, the correctly
// rounded division is taken, clamped to +-127 as the reference clamps.  For a
// normal s = amax/127 rounded, |x/s| < 127.5 for every x of the group, so the
// clamp never binds on the fast path, and |y| < 128 makes 4 ulp(y) <= 2^-15
// (the margin used, 2^-13, is four times that).  A denormal s (a group
// maximum below 127 * 2^-126) keeps less precision, |x/s| can pass 127.5 and
// the clamp binds: r = +inf sends every value of such a group to the
// division.  (Clamping before rounding equals rounding then clamping: +-127
// are integers and rounding is monotonic.)
__device__ __forceinline__ float q8_recip(float s) {
    return s >= 0x1p-126f ? __builtin_amdgcn_rcpf(s) : __builtin_inff();
}

__device__ __forceinline__ int q8_value_fast(float x, float s, float r) {
    const float y = x * r;
    float q = rintf(y);
    if (__builtin_expect(!(fabsf(y - q) < 0.5f - 0x1p-13f), 0)) q = rintf(fminf(fmaxf(x / s, -127.0f), 127.0f));
    return (int)q;
}

// runq.c:137: xt = s * 128 * sum(q), the bias-correction term of the
// unsigned-weight dot product.
__device__ __forceinline__ float q8_bias_term(float s, int sumq) {
    return s * 128.0f * (float)sumq;
}

// The batched-prefill GEMM operand of quantized activations [T][K]: xqp
// holds q in the MFMA chunk order (INT4 weights: per chunk of G/4 columns,
// the odd columns then the even ones; INT8: natural order) and rec [K/G][T]
// one 16-byte record per (group, token), pf_record.  Producers that
// quantize write it directly (xqp == nullptr: not wanted).
struct __attribute__((aligned(16))) PfRecord {
    int c;       // the MFMA accumulator input (every row of the token's column)
    float xs;    // the group's activation scale
    float xt;    // its bias term
    int pad;
};

struct PfOperand {
    int8_t* xqp;
    PfRecord* rec;
    int bits;
    int K;
    int T;
};

// The qkv GEMM's fused epilogue (EPI 1): rows [0, dim) are q, [dim, dim +
// kv_dim) k and the rest v of token t at position pos0 + t; q and k pairs
// (2i, 2i + 1) are rotated as k_rope_kv_append rotates them (runq.c:
// 351-365) — q stored to out, k and v appended to the caches — so no
// separate RoPE / append launch follows.  Token t is rotated for position
// pos0 + t and stored to cache row row0 + t (row0 = pos0 for the KV cache;
// 0 for a staging buffer of the chunk's rows).
struct PfRope {
    const float* rope;
    float* kcache;
    float* vcache;
    int pos0, dim, kv_dim, hs, max_t, k_il, row0;
};

// The record: xt = q8_bias_term(xs, sum(q)) (runq.c:137) and c =
// 128*sum(q), the MFMA's accumulator input, so that D = d + 128*sum(q)
// comes out of the MFMA.  INT4 weights enter the MFMA in offset binary
// (s4 + 8, see k_pf_gemm3), so there c = 120*sum(q) completes the same D.
__device__ __forceinline__ PfRecord pf_record(float xs, int sumq, int bits) {
    const int c = sumq * (bits == 4 ? 120 : 128);
    return PfRecord{c, xs, q8_bias_term(xs, sumq), 0};
}

// Emit element i of token t (i < K, K % G == 0) with value q and group scale
// s.  Every lane of the wave calls it together, with each group's G elements
// on G consecutive lanes; `in` false marks a lane past the end, which
// contributes 0 and stores nothing.
template <int G>
__device__ __forceinline__ void pf_emit(const PfOperand& p, int t, int i, int q, float s, bool in) {
    const int sum = group_isum<G>(in ? q : 0);   // exact in any order
    if (!in) return;
    constexpr int CH = G / 4;
    const int j = i % G;
    int pj = j;
    if (p.bits == 4) {
        const int jj = j % CH;
        pj = j - jj + ((jj & 1) ? jj / 2 : CH / 2 + jj / 2);
    }
    p.xqp[(size_t)t * p.K + (i - j + pj)] = (int8_t)q;
    if (j == 0) p.rec[(size_t)(i / G) * p.T + t] = pf_record(s, sum, p.bits);
}

// runq.c:155 for one group, as GCC -O3 -march=native compiles it (two FMAs):
//   sum = fma(ws, t, sum),  t = fma(xs, (float)d_u8, -xt),  d_u8 = d + 128*sum(q)
// d_u8 is the dot the reference's VPDPBUSD produces on +128-biased weights;
// with it every per-group term is bit-identical to the reference's.
__device__ __forceinline__ float group_term(float xs, float xt, int d, int sumq) {
    const int du8 = d + 128 * sumq;
    return __builtin_fmaf(xs, (float)du8, -xt);
}

// ---------------------------------------------------------------------------
// Dot products on v_dot4_i32_i8.

__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Split the activation bytes of one packed-int4 dword's columns into the
// even columns (x0,x2,x4,x6) and odd columns (x1,x3,x5,x7).  a = x0..x3,
// b = x4..x7 (little-endian bytes).  v_perm_b32 selects bytes of {b:a}.
__device__ __forceinline__ int even_bytes(int a, int b) {
    return (int)__builtin_amdgcn_perm((unsigned)b, (unsigned)a, 0x06040200u);
}
__device__ __forceinline__ int odd_bytes(int a, int b) {
    return (int)__builtin_amdgcn_perm((unsigned)b, (unsigned)a, 0x07050301u);
}

// Eight packed int4 weights (w) against eight activations given as their
// even/odd byte splits: the nibbles are moved into the high half of each
// byte, where they read as signed int8 values 16*q, and the dot is exact
// 16x the true one (|16*q*x| sums stay far below 2^31).
__device__ __forceinline__ int dot8_q4_x16(unsigned w, int xe, int xo, int c) {
    int hi = (int)(w & 0xF0F0F0F0u);          // 16 * odd columns
    int lo = (int)((w << 4) & 0xF0F0F0F0u);   // 16 * even columns
    return dot4(hi, xo, dot4(lo, xe, c));
}

// Index of element i of head g's key at position t in an fp32 K cache:
// row layout [n_kv][max_t][hs] (the op ABI's) or the engine's
// column-interleaved layout [n_kv][hs/4][max_t][4], in which float4 column
// f of consecutive positions is contiguous, so a wave that reads one
// position per lane reads one coalesced KiB per column.
__host__ __device__ inline size_t k_index(int il, int g, int t, int i, int hs, int max_t) {
    return il ? (((size_t)g * (hs >> 2) + (i >> 2)) * max_t + t) * 4 + (i & 3) : ((size_t)g * max_t + t) * hs + i;
}

}  // namespace l2q
