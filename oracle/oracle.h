/* oracle.h - CPU restatement of the reference decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the GPU path is compared
 * against (and the "port" CPU baseline); the product never links it.
 *
 * Every function restates the reference's arithmetic in plain C, with the
 * group size G as a parameter (the reference fixes G = 32, runq.c:26):
 *   orc_quantize_act   runq.c:117-139
 *   orc_matmul_q8      runq.c:142-159  (biased u8 weights, VNNI semantics)
 *   orc_matmul_q4      runq.c:142-159 applied to the int4 dequant of
 *                      tools/quantize_int4.py:38-51 (q4 lifted to the same
 *                      biased formula, so a QLL4 model lifted to QLL8 gives
 *                      the identical result through runq)
 *   orc_rmsnorm        runq.c:294-305  (16 accumulators + the reduce tree of
 *                      _mm512_reduce_add_ps)
 *   orc_softmax        runq.c:307-318
 *   orc_rope           runq.c:351-365
 *   orc_attention      runq.c:367-391
 *   orc_kv_quant       v5-cuda-fused/run.cu:204-249 (int8 KV cache row)
 *   orc_attention_kv8  v5-cuda-fused/run.cu:350-410 (attention over it; in
 *                      double, the value every float order approximates)
 *   orc_attention_kv8_ordered  the same in the GPU kernels' float order
 *   orc_attention_kv8_split    the same split over the context (the
 *                      split kernel's float order)
 *   orc_swiglu         runq.c:405-410
 *   orc_forward        runq.c:320-421
 * Floating-point contraction follows a GCC -O3 -march=native build of
 * runq.c: the loops the reference writes as `a += b*c` are explicit fmaf
 * here, everything else is compiled with -ffp-contract=off.
 */
#ifndef L2Q_ORACLE_H
#define L2Q_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void orc_quantize_act(const float* x, int n, int group, int8_t* xq, float* xs, float* xt);

/* out[rows]; w: biased u8 [rows][cols]; dots (optional): signed int32
 * group dots [rows][cols/group]. */
void orc_matmul_q8(float* out, const int8_t* xq, const float* xs, const float* xt,
                   const uint8_t* w, const float* ws, int rows, int cols, int group,
                   int32_t* dots);

/* Same with packed int4 weights [rows][cols/2]. */
void orc_matmul_q4(float* out, const int8_t* xq, const float* xs, const float* xt,
                   const uint8_t* w, const float* ws, int rows, int cols, int group,
                   int32_t* dots);

void orc_rmsnorm(float* o, const float* x, const float* w, int n);
void orc_softmax(float* x, int n);

/* RoPE of q (dim) and k (kv_dim) at `pos`, in place (runq.c:351-365). */
void orc_rope(float* q, float* k, int pos, int dim, int kv_dim, int hs);

/* One layer's attention (runq.c:367-391); position t of kv head g lives at
 * kc + g*head_stride + t*t_stride.  att_scratch: n_heads*att_stride floats,
 * att_stride > pos. */
void orc_attention(const float* q, const float* kc, const float* vc, float* out, int pos,
                   int n_heads, int n_kv_heads, int hs, size_t t_stride, size_t head_stride,
                   float* att_scratch, int att_stride);

/* One kv head's int8 cache row and its scale (v5-cuda-fused/run.cu:
 * 204-249). */
void orc_kv_quant(const float* row, int hs, int8_t* q, float* s);

/* Attention over an int8 KV cache (v5-cuda-fused/run.cu:350-410), in
 * double: row t of kv head g at kc + g*head_stride + t*t_stride, its scale
 * at ks[t*s_t_stride + g*s_head_stride]. */
void orc_attention_kv8(const float* q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
                       float* out, int pos, int n_heads, int n_kv_heads, int hs, size_t t_stride,
                       size_t head_stride, size_t s_t_stride, size_t s_head_stride);

/* orc_attention_kv8 in the float order of this build's GPU kernels (see
 * oracle.c), for bit-exact comparison; same arguments. */
void orc_attention_kv8_ordered(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                               const float* vs, float* out, int pos, int n_heads, int n_kv_heads, int hs,
                               size_t t_stride, size_t head_stride, size_t s_t_stride, size_t s_head_stride);

/* orc_attention_kv8 split over the context in S splits (S <= 64), in the
 * float order of this build's split kernel (see oracle.c); same arguments
 * plus S. */
void orc_attention_kv8_split(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                             const float* vs, float* out, int pos, int n_heads, int n_kv_heads, int hs,
                             size_t t_stride, size_t head_stride, size_t s_t_stride, size_t s_head_stride,
                             int S);

/* SwiGLU (runq.c:405-410); out may alias h. */
void orc_swiglu(float* out, const float* h, const float* h2, int n);

/* Model held by the oracle: pointers into a QLL tensor section. */
typedef struct orc_model orc_model;

/* cfg: dim, hidden, layers, heads, kv_heads, vocab (positive), seq_len. */
/* max_t (<= seq_len) sizes the KV cache; the cache stride does not
 * change any value, only memory use. */
orc_model* orc_model_create(const int cfg[7], const void* weights, size_t bytes,
                            int wbits, int group, int max_t);
void orc_model_free(orc_model* m);

/* Switch the model to the int8 KV cache (v5-cuda-fused/run.cu:41-48,
 * INT8_KV=1): each position's rotated k and v rows are stored through
 * orc_kv_quant and attention runs through orc_attention_kv8.  Returns 0, or
 * -1 when the caches cannot be allocated. */
int orc_model_set_kv8(orc_model* m, int on);

/* With the int8 KV cache: attention over more than `split_from` positions
 * in the split order with `splits` splits (orc_attention_kv8_split), over
 * fewer in orc_attention_kv8_ordered, as the GPU engine runs it; splits 0
 * (the default) keeps orc_attention_kv8_ordered everywhere.  Returns 0, or
 * -1 for splits outside 0..64. */
int orc_model_set_kv8_splits(orc_model* m, int splits, int split_from);

/* forward(token, pos) -> logits[vocab] (owned by the model).  If x_layers
 * is not NULL it receives the residual stream after the embedding and after
 * each layer ([n_layers+1][dim]). */
const float* orc_forward(orc_model* m, int token, int pos, float* x_layers);

/* Greedy decode: feed prompt[0..n_prompt), then sample argmax until
 * n_steps positions have run (no BOS stop).  ids_out[n_steps]: the token
 * chosen after each position (forced prompt tokens included). */
void orc_greedy(orc_model* m, const int* prompt, int n_prompt, int n_steps, int* ids_out);

/* First index of the maximum, runq.c:578-585. */
int orc_argmax(const float* v, int n);

/* y[i] = expf(x[i]) with the host C library (the reference's expf). */
void orc_expf_array(const float* x, float* y, size_t n);

/* RoPE (cos, sin) table, runq.c:351-356, [max_t][head_size/2][2]. */
void orc_rope_table(float* table, int max_t, int head_size);

#ifdef __cplusplus
}
#endif
#endif
