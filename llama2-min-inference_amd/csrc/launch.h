// launch.h - host-side launchers of the decode kernels (C++), shared by the
// op ABI (ops.hip) and the engine (engine.hip).  Each returns L2Q_OK or a
// negative status after recording a message with set_error().
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gemv.h"
#include "l2q.h"
#include "step_args.h"

namespace l2q {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int hip_fail(hipError_t e, const char* what);   // records and returns L2Q_ERR_HIP
int check_launch(const char* what);             // hipGetLastError after a launch

// GEMV: bits 4/8, group 32/64, prologue kPreq/kQuant/kNorm, epilogue
// kStore/kRopeKV/kSwiglu (see gemv.h).  Validates shapes and alignment.
int launch_gemv_fused(int bits, int group, int pro, int epi, const GemvArgs& a, hipStream_t st);
int launch_gemv(int bits, int group, const GemvArgs& a, hipStream_t st);   // kPreq + kStore

// pf (optional): also write the batched-prefill GEMM operand (PfOperand,
// device.h), replacing launch_pf_prep; xq may then be null.
int launch_quantize(const float* x, int n, int group, int8_t* xq, float* xs, hipStream_t st,
                    const PfOperand* pf = nullptr);

// emb/meta: layer-0 form (x = emb[meta[0]]); otherwise x.
// T > 1: T consecutive vectors of n (x, resid, xout, xq rows of n; xs rows of n/group).
// pf: the prefill GEMM operand form (k_pf_rmsnorm_quant): the operand is the
// only quantized output (xq, xs, emb null), pointers 16-byte aligned.
int launch_rmsnorm_quant(const float* x, const float* emb, const int* meta, const float* resid,
                         float* xout, const float* w, int n, int group, int8_t* xq, float* xs,
                         hipStream_t st, int T = 1, const PfOperand* pf = nullptr);

int launch_swiglu_quant(const float* hb, const float* hb2, int n, int group, int8_t* xq, float* xs,
                        float* gout, hipStream_t st);

// T > 1: tokens at positions pos..pos+T-1, their q/k/v rows `stride` floats apart.
int launch_rope_kv_append(float* q, const float* k, const float* v, float* kcache, float* vcache,
                          const float* rope, const int* meta, int pos, int dim, int kv_dim, int hs,
                          int max_t, hipStream_t st, int T = 1, int stride = 0, int k_il = 0);

// Split-context attention (tolerance path): S splits per head, partial
// buffers of n_heads*S*hs and n_heads*S*2 floats.
int launch_attention_split(const float* q, const float* kcache, const float* vcache, float* out, float* part_o,
                           float* part_ml, int S, const int* meta, int pos, int n_heads, int n_kv_heads, int hs,
                           int max_t, hipStream_t st);

// Split-context attention in one kernel (the engine's tolerance mode):
// S splits per head (attention_flash_splits), partials of
// attention_flash_part_floats floats and n_heads zeroed counters that the
// kernel leaves zeroed; K in the layout k_il (see k_index).
// int8-KV attention split over the context (S splits, partials and zeroed
// counters as launch_attention_flash); kst/vst: the step's staged rows to
// append at pos (or both null).
// nq > 1: queries pos.. of a batch (q, out rows at the given strides), each
// with its own attention_flash_part_floats partials and n_heads counters.
int launch_attention_kv8_split(const float* q, const float* kst, const float* vst, int8_t* k8, int8_t* v8,
                               float* ks, float* vs, float* out, float* part, unsigned* cnt, int S, const int* meta,
                               int pos, int n_heads, int n_kv_heads, int hs, int max_t, hipStream_t st, int nq = 1,
                               int q_stride = 0, int out_stride = 0);
bool attention_flash_ok(int hs);
int attention_flash_splits(int n_heads, int max_t, int ncu);
size_t attention_flash_part_floats(int n_heads, int S, int hs);
int launch_attention_flash(const float* q, const float* kcache, const float* vcache, float* out, float* part,
                           unsigned* cnt, int S, const int* meta, int pos, int n_heads, int n_kv_heads, int hs,
                           int max_t, int k_il, hipStream_t st);

// Attention in the reference's exact order: `scores` is n_heads*max_t
// floats of scratch, S the number of score workgroups per head.
// T > 1: queries at positions pos..pos+T-1 (causal), q rows `q_stride` floats
// apart, outputs [T][n_heads*hs], scores [T][n_heads][max_t].
// k_il: the K cache's layout (see k_index).
// A single query (T == 1) runs as one kernel (k_attn_fused, same operations)
// when `fused` is 1, or when it is -1, meta is NULL, the head size has a
// fused form and pos + 1 <= attention_fused_max(); otherwise as two.
int launch_attention_exact(const float* q, const float* kcache, const float* vcache, float* out, float* scores,
                           int S, const int* meta, int pos, int n_heads, int n_kv_heads, int hs, int max_t,
                           hipStream_t st, int T = 1, int q_stride = 0, int fused = -1, int k_il = 0);
bool attention_exact_ok(int max_t);
int attention_exact_max();   // the longest cache attention_exact_ok accepts
bool attention_fused_ok(int hs);
// Longest context served by the one-kernel form: every context the exact
// path takes (measured faster than the pair at 64..4096 positions with the
// engine's K layout; L2Q_ATTN_FUSED_MAX lowers it, for measurements).
int attention_fused_max();

// int8 KV cache: append one position / attention over positions 0..pos.
bool kv8_shape_ok(int n_heads, int n_kv_heads, int hs, int max_t);
// nrows > 1: rows [n_kv][src_rows][hs] of k / v (the first nrows of each
// head) to positions pos.. (no meta).
int launch_kv8_append(const float* k, const float* v, int8_t* k8, int8_t* v8, float* ks, float* vs,
                      const float* rope, const int* meta, int pos, int n_kv_heads, int hs, int max_t,
                      hipStream_t st, int nrows = 1, int src_rows = 1);
// The one-kernel int8-cache attention (k_attn8_fused).  With kst / vst (the
// step's rotated k and v rows, [n_kv][hs]) it first appends position pos to
// the caches (the k_kv8_append operations); without them it only reads.
int launch_attention_kv8(const float* q, int8_t* k8, int8_t* v8, float* ks, float* vs, float* out, float* scores,
                         const int* meta, int pos, int n_heads, int n_kv_heads, int hs, int max_t, hipStream_t st,
                         const float* kst = nullptr, const float* vst = nullptr, int nq = 1, int q_stride = 0,
                         int out_stride = 0);

// Score workgroups for n positions: ~128 positions each, at most 64.
inline int score_splits(int n) {
    const int S = (n + 127) / 128;
    return S < 1 ? 1 : (S > 64 ? 64 : S);
}

// Batched prefill (prefill.h): activation preparation and the exact-fold GEMM.
constexpr int kPfMaxTokens = 128;    // tokens per prefill chunk
int launch_pf_prep(int bits, int group, const int8_t* xq, const float* xs, int K, int T, int8_t* xqp, PfRecord* rec,
                   hipStream_t st);
// rope (optional): the qkv form, q rotated to out, k and v appended to the caches (PfRope).
// swiglu (optional): the w1|w3 form, SwiGLU + Q8 straight into the w2 operand (out unused).
int launch_pf_gemm(int bits, int group, const void* w, const float* ws, int rows, int cols, const int8_t* xqp,
                   const PfRecord* rec, int T, float* out, int ldo, hipStream_t st, const PfRope* rope = nullptr,
                   const PfOperand* swiglu = nullptr);
// The prefill's attention of T > 1 queries (exact order): scores, softmax,
// p*V and (pf set) the Q8 operand of the wo GEMM in one kernel where the
// shape allows it (head size 64 / 128, groups inside a head, a context of at
// most 256 positions), else the three-kernel batched path and the quantize.
// out [T][dim] is written only without pf.
int launch_attention_prefill(const float* q, const float* kcache, const float* vcache, float* out, float* scores,
                             int pos, int n_heads, int n_kv_heads, int hs, int max_t, hipStream_t st, int T,
                             int q_stride, int k_il, int group, const PfOperand* pf);
int launch_pf_embed(const float* emb, const int* tokens, float* x, int dim, int T, hipStream_t st);

int launch_argmax(const float* v, int n, int* out, hipStream_t st);

// The one-kernel decode step (step.h): whether it is built for this shape;
// bytes of its LDS layout; raising its LDS limit to `lds` and reporting how
// many of its workgroups fit on one CU; one launch of `grid` workgroups.
bool step_shape_ok(int d, int h, int hs);
size_t step_lds_bytes();
int step_prepare(size_t lds, int* per_cu);
int launch_step_kernel(const StepArgs& a, int grid, size_t lds, hipStream_t st);
int launch_unbias(const uint8_t* src, int8_t* dst, size_t n, hipStream_t st);

// Shape checks shared by the op ABI and the engine.
bool gemv_shape_ok(int bits, int group, int rows, int cols);
bool attention_shape_ok(int n_heads, int n_kv_heads, int hs);

}  // namespace l2q
