/* l2q.h - C ABI of the MI355X batch-1 quantized Llama-2 decode path.
 *
 * Two layers of entry points, all plain C types (no torch, no HIP types):
 *
 *   Engine ABI - what the host runner calls once per position.  It replaces
 *   the reference's single seam, `float* forward(Transformer*, int token,
 *   int pos)` (v1-int8-vnni/runq.c:320), together with its GPU counterparts
 *   `forward_step` (v3-cuda-kvcache/run.cu:422) and `run_token`
 *   (v5-cuda-fused/run.cu:682-695).
 *
 *   Op ABI - one GPU op per call, device pointers in, device pointers out,
 *   enqueued on a caller-supplied HIP stream (passed as `void*`; NULL is the
 *   null stream).  These replace the reference's kernel launchers
 *   (`launch_matmul` v5-cuda-fused/run.cu:584, `launch_rmsnorm_quant` :590,
 *   `launch_quant` v3-cuda-kvcache/run.cu:403) and are what the parity and
 *   microbenchmark harnesses drive.
 *
 * Every function returns L2Q_OK (0) or a negative status; l2q_last_error()
 * then returns a human-readable message (thread-local).  The library never
 * calls exit(); the runner maps a failure to the reference's fail-fast exit
 * (runq.c:258-275, v5-cuda-fused/run.cu:50-52).
 *
 * Device scratch: l2q_attention, l2q_attention_ex, l2q_attention_split and
 * l2q_gemm_q keep their intermediates (per-head scores, split partials,
 * permuted activations) in one library-owned buffer per GPU, grown on
 * demand (growing synchronizes the device).  They return before the GPU
 * work ends, so calls from different host threads or on different streams
 * of one GPU must not overlap: issue them from one thread on one stream.
 * The engine owns its own buffers and is not affected.
 *
 * Quantization conventions shared by every entry point:
 *   - a "group" is G consecutive elements of one row (G = 32 for reference
 *     files, 64 for the Llama-2-7B configurations);
 *   - activations are Q8: int8 q in [-127,127] plus one fp32 scale per group,
 *     s = amax/127 (1e-8 if amax == 0), q = round-half-even(x/s)
 *     (runq.c:117-139);
 *   - INT8 weights are signed int8 (the on-disk +128 bias removed),
 *     row-major [rows][cols], scales [rows][cols/G];
 *   - INT4 weights are packed two per byte, low nibble = even column,
 *     two's complement, [rows][cols/2], scales [rows][cols/G]
 *     (tools/quantize_int4.py:38-51).
 */
#ifndef L2Q_H
#define L2Q_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define L2Q_OK              0
#define L2Q_ERR_ARG        -1   /* bad argument or unsupported shape        */
#define L2Q_ERR_HIP        -2   /* a HIP runtime call failed                */
#define L2Q_ERR_FORMAT     -3   /* weights image too short / inconsistent   */
#define L2Q_ERR_NOMEM      -4   /* device allocation failed                 */
#define L2Q_ERR_STATE      -5   /* engine used out of order (pos > max)     */

/* Model hyper-parameters, byte-identical to the 7 x int32 header of the
 * reference checkpoints (runq.c:33-41, v5-cuda-fused/run.cu:57-59).
 * vocab_size is passed positive; the checkpoint's sign convention (negative
 * = unshared classifier) is resolved by the reader. */
typedef struct {
    int dim;
    int hidden_dim;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int vocab_size;
    int seq_len;
} l2q_config;

/* ------------------------------------------------------------------------
 * Errors / device
 * ---------------------------------------------------------------------- */

/* Message for the last failing call on this thread ("" if none). */
const char* l2q_last_error(void);

/* Number of visible HIP devices (0 when none); never fails. */
int l2q_device_count(void);

/* ------------------------------------------------------------------------
 * Engine ABI
 * ---------------------------------------------------------------------- */

typedef struct l2q_engine l2q_engine;

/* Build an engine from a checkpoint's tensor section.
 *
 * `weights` points at the first byte after the file header (the token
 * embedding table) of a QLL8 (wbits = 8) or QLL4 (wbits = 4) checkpoint,
 * usually inside the caller's mmap; `weights_bytes` is how many bytes are
 * readable there.  Tensor order and sizes follow runq.c:230-253 /
 * v5-cuda-fused/run.cu:534-551 with `group` elements per scale.  The engine
 * copies everything it needs to the current device (one allocation, laid out
 * for the kernels), so the caller may unmap afterwards.
 *
 * `max_steps` sizes the KV cache (positions 0..max_steps-1), as the GPU
 * reference runners do (v5-cuda-fused/run.cu:1147-1150); it is clamped to
 * cfg->seq_len, and a cache of more than 4096 positions (the exact-order
 * attention's limit; Llama-2's seq_len is 4096) is L2Q_ERR_ARG.  Replaces read_checkpoint/memory_map_weights/
 * malloc_run_state (runq.c:190-283) and load_weights/alloc_state/build_graph
 * (v5-cuda-fused/run.cu:534-582, 671-679). */
int l2q_engine_create(const l2q_config* cfg, const void* weights,
                      size_t weights_bytes, int wbits, int group,
                      int max_steps, l2q_engine** out);

/* Batched prefill: positions pos0..pos0+n-1 take tokens[0..n) through every
 * layer together (chunks of up to 128 tokens; the weights stream once per
 * chunk, group dots on int8 MFMA), leaving the KV cache exactly as n calls
 * of l2q_engine_forward would; if logits is not NULL it receives the logits
 * of the last position, bit-identical to l2q_engine_forward's (also with
 * L2Q_ENGINE_KV_INT8: the rows are appended and each query attends as its
 * decode step would).  Replaces the prompt-forcing loop of generate()
 * (runq.c:695-700, v5-cuda-fused/run.cu:969-974) and the batched forward of
 * v2-cuda/run.cu:347-394. */
int l2q_engine_prefill(l2q_engine* e, const int* tokens, int n, int pos0,
                       float* logits);

/* Engine options (l2q_engine_create_ex). */
#define L2Q_ENGINE_KV_INT8 1   /* int8 KV cache (l2q_kv8_append semantics), the
                                  reference's -DINT8_KV=1 build; its attention
                                  is l2q_attention_kv8's (one workgroup per
                                  head) up to L2Q_KV8_SPLIT_FROM positions and
                                  l2q_attention_kv8_ex's split form (with
                                  l2q_engine_attention_splits splits) beyond */
#define L2Q_KV8_SPLIT_FROM 1024
#define L2Q_ENGINE_STEP_KERNEL 2   /* run each decode step as one persistent
                                  kernel with grid barriers between its phases
                                  where the shape allows it (see
                                  l2q_engine_uses_step_kernel) instead of the
                                  graph of one kernel per op (v5-cuda-fused/
                                  run.cu:600-679's op sequence); same bits.
                                  Opt-in: slower than the graph on MI355X
                                  today.  No counterpart in the reference. */

#define L2Q_ENGINE_ATTN_SPLIT 4   /* tolerance mode: decode attention split over
                                  the context in one kernel (per-split softmax
                                  partials merged in split order), with the
                                  fp32 cache; equal to the reference's
                                  attention up to rounding (relative error
                                  ~1e-6), not bit for bit, from
                                  L2Q_ATTN_SPLIT_FROM positions on (shorter
                                  contexts run the exact one-kernel attention,
                                  the faster there).  The default is the
                                  reference's exact order (runq.c:367-391).
                                  head_size 48, 64 or 128; not with
                                  L2Q_ENGINE_KV_INT8.  No counterpart in the
                                  reference. */

#define L2Q_ATTN_SPLIT_FROM 320   /* positions from which L2Q_ENGINE_ATTN_SPLIT
                                     splits the attention */

/* l2q_engine_create with option flags (0 gives l2q_engine_create). */
int l2q_engine_create_ex(const l2q_config* cfg, const void* weights,
                         size_t weights_bytes, int wbits, int group,
                         int max_steps, int flags, l2q_engine** out);

/* One decode step: embed `token`, run every layer at position `pos`
 * (appending its K/V), final norm and classifier.  If `logits` is not NULL
 * the vocab_size fp32 logits are copied into it (host memory).  Synchronous.
 * Positions must be fed in order 0,1,2,... as in the reference loops
 * (runq.c:697-711); pos >= max_steps is L2Q_ERR_STATE.
 * Replaces forward() (runq.c:320-421) and run_token() (v5:682-695). */
int l2q_engine_forward(l2q_engine* e, int token, int pos, float* logits);

/* Same step, but the greedy choice (first index of the maximum logit,
 * sample_argmax runq.c:578-585) is made on the device and only the index
 * crosses to the host. */
int l2q_engine_forward_argmax(l2q_engine* e, int token, int pos, int* next);

/* Diagnostic step that runs the same kernels one launch at a time (no
 * graph) and copies the residual stream after the embedding and after every
 * layer into `x_layers` ([n_layers + 1][dim] fp32, host) and, if not NULL,
 * the logits.  Used for per-layer parity checks. */
int l2q_engine_forward_debug(l2q_engine* e, int token, int pos,
                             float* x_layers, float* logits);

/* Replay the captured step `n_steps` times at positions pos0 .. pos0+n-1
 * with token ids `tokens` (host array, length n_steps), without copying
 * logits back, and report the elapsed device time in milliseconds measured
 * with HIP events on the engine's stream.  Benchmark entry point. */
int l2q_engine_time_steps(l2q_engine* e, const int* tokens, int pos0,
                          int n_steps, double* elapsed_ms);

/* Benchmark entry: launch the step's GEMV kernel of one matrix kind
 * `n_launches` times back to back on the engine's stream, with the decode's
 * own arguments (prologue, epilogue, weights of layer i % n_layers, so the
 * launches rotate over every layer's weights), and report the elapsed device
 * time in milliseconds (HIP events).  Inputs are the engine's current
 * activations; outputs go to a scratch area, so the decode state is left
 * unchanged.  The reference has no counterpart (its kernels are timed by the
 * whole step, v5-cuda-fused/run.cu:10-11). */
#define L2Q_GEMV_QKV        0   /* wq|wk|wv: RMSNorm prologue, RoPE + KV append epilogue */
#define L2Q_GEMV_WO         1   /* wo: Q8 quantize prologue */
#define L2Q_GEMV_W13        2   /* w1|w3: RMSNorm prologue, SwiGLU epilogue */
#define L2Q_GEMV_W2         3   /* w2: Q8 quantize prologue */
#define L2Q_GEMV_CLASSIFIER 4   /* wcls: final RMSNorm prologue */
int l2q_engine_time_gemv(l2q_engine* e, int kind, int n_launches, double* elapsed_ms);

/* The number of context splits of the engine's decode attention when it
 * runs split over the context (L2Q_ENGINE_KV_INT8 beyond L2Q_KV8_SPLIT_FROM
 * positions: the order of the oracle's orc_attention_kv8_split with this
 * many splits; L2Q_ENGINE_ATTN_SPLIT), 0 when it runs the reference's exact
 * order.
 * Chosen at creation from the head count, the cache length and the GPU's CU
 * count.  No counterpart in the reference. */
int l2q_engine_attention_splits(const l2q_engine* e);

/* 1 when the engine runs each decode step as one persistent kernel
 * (L2Q_ENGINE_STEP_KERNEL was given and the shape has it: INT4 group 64, the
 * Llama-2-7B row shapes, head size 128, fp32 KV cache, one workgroup resident
 * per CU), 0 when it runs the per-op kernel graph.  Both give the same bits.
 * No counterpart in the reference. */
int l2q_engine_uses_step_kernel(const l2q_engine* e);

/* Device bytes held by the engine (weights + KV cache + activations). */
size_t l2q_engine_device_bytes(const l2q_engine* e);

void l2q_engine_destroy(l2q_engine* e);

/* ------------------------------------------------------------------------
 * Op ABI (device pointers, asynchronous on `stream`)
 * ---------------------------------------------------------------------- */

/* Q8 activation quantize of x[n] into xq[n], xs[n/group].
 * runq.c:117-139 (quantize_act), v3-cuda-kvcache/run.cu:104-129. */
int l2q_quantize_act(const float* x, int n, int group,
                     int8_t* xq, float* xs, void* stream);

/* INT8 GEMV: out[r] = sum_b ws[r,b] * (xs[b]*(d_b(r) + 128*sum_b(xq)) - xt[b])
 * with d_b(r) = sum_{j<group} w[r, b*group+j] * xq[b*group+j] the exact
 * int32 group dot and xt[b] = xs[b]*128*sum_b(xq): the reference's formula
 * for its +128-biased weights, folded over b in order with FMAs, so out is
 * bit-identical to runq.c:142-159 (matmul_q8; v3-cuda-kvcache/run.cu:177-202
 * is the GPU counterpart).  If `dots` is not NULL the int32 group dots are
 * written to dots[r*(cols/group) + b].  w is signed int8 [rows][cols];
 * rows of at most 12 KiB (cols*bits/8 <= 12288). */
int l2q_gemv_q8(float* out, const int8_t* xq, const float* xs,
                const int8_t* w, const float* ws, int rows, int cols,
                int group, int32_t* dots, void* stream);

/* INT4 GEMV, same contract with w packed [rows][cols/2] (low nibble = even
 * column, two's complement): the dequant of tools/quantize_int4.py:38-51
 * through the formula above (the result equals runq's on the model with
 * every int4 value stored as int8).  v5-cuda-fused/run.cu:252-330 is the
 * GPU counterpart. */
int l2q_gemv_q4(float* out, const int8_t* xq, const float* xs,
                const uint8_t* w, const float* ws, int rows, int cols,
                int group, int32_t* dots, void* stream);

/* Remove the +128 bias of on-disk QLL8 weights (u8 -> s8), n bytes.
 * v3-cuda-kvcache/run.cu:167-175. `dst` may equal `src`. */
int l2q_unbias_q8(const uint8_t* src, int8_t* dst, size_t n, void* stream);

/* Fused residual-add + RMSNorm + Q8 quantize of one vector of n floats:
 *   v = x + (resid ? resid : 0);  if (xout) xout = v;
 *   o = w * (inv * v), inv = 1/sqrtf(sum(v^2)/n + 1e-5f);  quantize(o).
 * runq.c:294-305 (rmsnorm) + :117-139, v5-cuda-fused/run.cu:120-175. */
int l2q_rmsnorm_quant(const float* x, const float* resid, float* xout,
                      const float* w, int n, int group,
                      int8_t* xq, float* xs, void* stream);

/* SwiGLU + Q8 quantize: g = hb * (1/(1+expf(-hb))) * hb2 over n elements.
 * runq.c:404-412, v5-cuda-fused/run.cu:180-200.  If `gout` is not NULL the
 * fp32 product is stored there as well. */
int l2q_swiglu_quant(const float* hb, const float* hb2, int n, int group,
                     int8_t* xq, float* xs, float* gout, void* stream);

/* RoPE on q (all heads) and k, then append k and v at position `pos` of
 * one layer's cache.  `rope` is the [max_t][head_size/2][2] (cos, sin)
 * table from l2q_rope_table (device copy).  q is rotated in place.
 * Cache layout: [n_kv_heads][max_t][head_size] fp32 for K and for V.
 * runq.c:340-365, v5-cuda-fused/run.cu:332-345, 413-439. */
int l2q_rope_kv_append(float* q, const float* k, const float* v,
                       float* kcache, float* vcache, const float* rope,
                       int pos, int n_heads, int n_kv_heads, int head_size,
                       int max_t, void* stream);

/* Single-query multi-head attention over positions 0..pos of one layer's
 * cache (layout as above): out[h*hs + i] = sum_t softmax_t(q_h.k_t /
 * sqrtf(hs)) v_t[i], kv head = h / (n_heads/n_kv_heads).  Evaluated in the
 * reference's order (serial dot per position, expf identical to the host
 * C library's, serial softmax sum, serial p*V accumulation per element), so
 * the output is bit-identical to runq.c:367-391 (+ softmax :307-318).
 * max_t <= 4096 (the probabilities of a head are staged in LDS). */
int l2q_attention(const float* q, const float* kcache, const float* vcache,
                  float* out, int pos, int n_heads, int n_kv_heads,
                  int head_size, int max_t, void* stream);

/* l2q_attention with options (no reference counterpart: the engine's own
 * cache layout and the choice of kernels, for tests and measurements).
 * L2Q_ATTN_K_INTERLEAVED: kcache in the engine's column-interleaved layout
 * [n_kv_heads][head_size/4][max_t][4] (float4 column f of consecutive
 * positions contiguous) instead of [n_kv_heads][max_t][head_size].
 * L2Q_ATTN_ONE_KERNEL / L2Q_ATTN_TWO_KERNELS force the single-kernel form
 * (head sizes 48, 64, 128) or the scores + softmax/p*V pair; by default the
 * single kernel serves contexts up to a measured threshold.  Every form
 * gives the same bits.  L2Q_ATTN_SPLIT_CONTEXT instead runs the engine's
 * tolerance-mode form (L2Q_ENGINE_ATTN_SPLIT: the context split over about
 * two workgroups per CU in one kernel, head sizes 48, 64, 128), equal to
 * the exact result up to rounding; its partials and per-head counters live
 * in per-GPU library buffers, so calls that overlap on one GPU race. */
#define L2Q_ATTN_K_INTERLEAVED 1
#define L2Q_ATTN_ONE_KERNEL 2
#define L2Q_ATTN_TWO_KERNELS 4
#define L2Q_ATTN_SPLIT_CONTEXT 8
int l2q_attention_ex(const float* q, const float* kcache, const float* vcache,
                     float* out, int pos, int n_heads, int n_kv_heads,
                     int head_size, int max_t, int flags, void* stream);

/* The same attention split over the context (flash-decoding: per-split
 * online softmax, then a merge), for throughput; float results agree with
 * l2q_attention to ~1e-6 relative, not bit for bit.
 * v5-cuda-fused/run.cu:441-499 semantics. */
int l2q_attention_split(const float* q, const float* kcache, const float* vcache,
                        float* out, int pos, int n_heads, int n_kv_heads,
                        int head_size, int max_t, void* stream);

/* l2q_attention_split without any device allocation, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments, kernels and results as l2q_attention_split; its partials live
 * in a static per-GPU scratch array of 2^20 floats (4 MiB, held until the
 * process ends), so n_heads * splits * (head_size + 2) must fit in it
 * (splits = ceil((pos + 1) / 128), at most 512); larger calls return
 * L2Q_ERR_ARG.  Every call on one GPU shares that array: calls that overlap
 * on one GPU (other streams or threads) race and must be serialized by the
 * caller. */
int l2q_attention_split_noalloc(const float* q, const float* kcache, const float* vcache,
                                float* out, int pos, int n_heads, int n_kv_heads,
                                int head_size, int max_t, void* stream);

/* Batched GEMV of T activation vectors (a GEMM): out[t][r] = the row-r
 * output of l2q_gemv_q8 / l2q_gemv_q4 for input t, bit for bit, for
 * t < T.  xq [T][cols] int8 and xs [T][cols/group] as l2q_quantize_act
 * writes them per vector; w, ws as for the GEMVs; out [T][rows].  Group
 * dots on int8 MFMA.  Replaces launch_matmul with T > 1
 * (v2-cuda/run.cu:131-162, 390-395). */
int l2q_gemm_q(int wbits, float* out, const int8_t* xq, const float* xs,
               const void* w, const float* ws, int rows, int cols, int group,
               int T, void* stream);

/* ---- int8 KV cache (v5-cuda-fused/run.cu:41-48, built there with
 * -DINT8_KV=1) ----
 * Layout: kcache8 / vcache8 [n_kv_heads][max_t][head_size] int8, one fp32
 * scale per (kv head, position): kscale / vscale [n_kv_heads][max_t].
 * head_size % 16 == 0, head_size <= 256. */

/* Append position `pos`: k (n_kv_heads*head_size floats, rotated here with
 * `rope` when it is not NULL, as l2q_rope_kv_append rotates) and v are
 * quantized per kv head: s = amax/127 (1e-8 when 0), q = clamp(rint(x/s),
 * -127, 127).  Replaces kv_quant_kernel (v5-cuda-fused/run.cu:204-249). */
int l2q_kv8_append(const float* k, const float* v, int8_t* kcache8, int8_t* vcache8,
                   float* kscale, float* vscale, const float* rope, int pos,
                   int n_kv_heads, int head_size, int max_t, void* stream);

/* Attention over positions 0..pos of an int8 cache: score_t = (q_h.k8_t) /
 * sqrtf(hs) * kscale_t, softmax, out = sum_t p_t * vscale_t * v8_t.  Float
 * results within 1e-5 relative of the same formula in double (the
 * reference's own float order is a warp reduction, so no order is
 * canonical).  Replaces attention_cache_kernel (v5-cuda-fused/run.cu:
 * 350-410), which also quantizes its output; here the output stays fp32
 * and the next GEMV's prologue quantizes it.  max_t <= 8192. */
int l2q_attention_kv8(const float* q, const int8_t* kcache8, const int8_t* vcache8,
                      const float* kscale, const float* vscale, float* out, int pos,
                      int n_heads, int n_kv_heads, int head_size, int max_t, void* stream);

/* l2q_attention_kv8 with options.  flags 0 is l2q_attention_kv8 (one
 * workgroup per head).  L2Q_ATTN_SPLIT_CONTEXT splits the context over about
 * two workgroups per CU (the int8-KV engine's form): per-split softmax
 * partials merged in split order by the last workgroup of each head, a
 * fixed float order of its own (restated by the oracle's
 * orc_attention_kv8_split), within the same 1e-5 of the double formula;
 * partials and per-head counters in per-GPU library buffers, so calls that
 * overlap on one GPU race.  No counterpart in the reference. */
int l2q_attention_kv8_ex(const float* q, const int8_t* kcache8, const int8_t* vcache8,
                         const float* kscale, const float* vscale, float* out, int pos,
                         int n_heads, int n_kv_heads, int head_size, int max_t, int flags,
                         void* stream);

/* Greedy argmax on the device: out[0] = the first index of the maximum of
 * v[0..n), v 16-byte aligned (sample_argmax, runq.c:578-585; the engine's
 * l2q_engine_forward_argmax runs it inside its step).  As the reference's
 * scan from v[0]: NaNs are never taken, a NaN at index 0 gives 0, and so
 * does a vector of -inf. */
int l2q_argmax(const float* v, int n, int* out, void* stream);

/* expf exactly as the host C library computes it (the exp used by the
 * attention softmax and SwiGLU above), elementwise over n floats.  Exposed
 * so its identity with the host's expf can be checked on every input. */
int l2q_expf(const float* x, float* y, size_t n, void* stream);

/* Host helper: fill the RoPE (cos, sin) table for positions 0..max_t-1 with
 * the reference's float expressions (runq.c:351-356), so that device and
 * CPU rotations are bit-identical.  `table` has max_t*head_size floats. */
void l2q_rope_table(float* table, int max_t, int head_size);

#ifdef __cplusplus
}
#endif
#endif /* L2Q_H */
