/* oracle.c - CPU restatement of the reference decode path (test
 * infrastructure only; see oracle.h for what each function follows). */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* runq.c:117-139: per group amax, s = amax/127 (1e-8 when 0),
 * q = clamp(lrintf(x/s), +-127), xt = s*128*sum(q). */
void orc_quantize_act(const float* x, int n, int group, int8_t* xq, float* xs, float* xt) {
    for (int b = 0; b < n / group; b++) {
        const float* xb = x + (size_t)b * group;
        float amax = 0.0f;
        for (int j = 0; j < group; j++) { float a = fabsf(xb[j]); if (a > amax) amax = a; }
        float s = amax / 127.0f;
        if (s == 0.0f) s = 1e-8f;
        int sum = 0;
        for (int j = 0; j < group; j++) {
            int q = (int)lrintf(xb[j] / s);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            xq[(size_t)b * group + j] = (int8_t)q;
            sum += q;
        }
        xs[b] = s;
        if (xt) xt[b] = s * 128.0f * (float)sum;
    }
}

/* runq.c:150-156 per group: d = sum(u8 w * q x) (VPDPBUSD), then
 * sum += ws*(xs*d - xt), which GCC -O3 -march=native contracts into two
 * FMAs. */
static inline float group_accumulate(float sum, float ws, float xs, float xt, int d_u8) {
    return fmaf(ws, fmaf(xs, (float)d_u8, -xt), sum);
}

void orc_matmul_q8(float* out, const int8_t* xq, const float* xs, const float* xt,
                   const uint8_t* w, const float* ws, int rows, int cols, int group,
                   int32_t* dots) {
    const int nb = cols / group;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < rows; i++) {
        const uint8_t* wp = w + (size_t)i * cols;
        const float* wsr = ws + (size_t)i * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            int d = 0, sq = 0;
            for (int j = 0; j < group; j++) {
                d += (int)wp[b * group + j] * (int)xq[b * group + j];
                sq += xq[b * group + j];
            }
            if (dots) dots[(size_t)i * nb + b] = d - 128 * sq;
            sum = group_accumulate(sum, wsr[b], xs[b], xt[b], d);
        }
        out[i] = sum;
    }
}

/* tools/quantize_int4.py:47-50: byte j of a row holds column 2j in its low
 * nibble and column 2j+1 in its high nibble, both two's complement. */
void orc_matmul_q4(float* out, const int8_t* xq, const float* xs, const float* xt,
                   const uint8_t* w, const float* ws, int rows, int cols, int group,
                   int32_t* dots) {
    const int nb = cols / group;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < rows; i++) {
        const uint8_t* wp = w + (size_t)i * (cols / 2);
        const float* wsr = ws + (size_t)i * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* g = wp + (size_t)b * (group / 2);
            const int8_t* x = xq + (size_t)b * group;
            int d = 0, sq = 0;
            for (int j = 0; j < group / 2; j++) {
                int lo = (int8_t)(uint8_t)(g[j] << 4) >> 4;
                int hi = (int8_t)g[j] >> 4;
                d += lo * x[2 * j] + hi * x[2 * j + 1];
                sq += x[2 * j] + x[2 * j + 1];
            }
            if (dots) dots[(size_t)i * nb + b] = d;
            /* the same value runq's unsigned dot would give for q + 128 */
            sum = group_accumulate(sum, wsr[b], xs[b], xt[b], d + 128 * sq);
        }
        out[i] = sum;
    }
}

/* runq.c:294-305.  The reference accumulates x*x in 16 FMA lanes
 * (lane l takes j = l, l+16, ...), reduces them with _mm512_reduce_add_ps
 * (halves 8, 4, then pairs (0,2),(1,3), then (0,1)) and adds the tail. */
void orc_rmsnorm(float* o, const float* x, const float* w, int n) {
    float acc[16] = {0};
    int j = 0;
    for (; j + 16 <= n; j += 16)
        for (int l = 0; l < 16; l++) acc[l] = fmaf(x[j + l], x[j + l], acc[l]);
    float a8[8], a4[4];
    for (int l = 0; l < 8; l++) a8[l] = acc[l + 8] + acc[l];
    for (int l = 0; l < 4; l++) a4[l] = a8[l + 4] + a8[l];
    float p0 = a4[0] + a4[2], p1 = a4[1] + a4[3];
    float s = p0 + p1;
    /* tail (< 16 elements): GCC vectorises a block of 8 without fusing,
     * then contracts the scalar remainder */
    if (n - j >= 8)
        for (int e = 0; e < 8; e++, j++) s = s + x[j] * x[j];
    for (; j < n; j++) s = fmaf(x[j], x[j], s);
    s = 1.0f / sqrtf(s / n + 1e-5f);
    for (int i = 0; i < n; i++) o[i] = w[i] * (s * x[i]);
}

void orc_softmax(float* x, int n) {
    float m = x[0];
    for (int i = 1; i < n; i++) if (x[i] > m) m = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); sum += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

int orc_argmax(const float* v, int n) {
    int best = 0;
    float m = v[0];
    for (int i = 1; i < n; i++) if (v[i] > m) { m = v[i]; best = i; }
    return best;
}

/* runq.c:351-356: freq = 1/powf(10000, hd/hs), angle = pos*freq. */
void orc_rope_table(float* table, int max_t, int head_size) {
    for (int pos = 0; pos < max_t; pos++)
        for (int hd = 0; hd < head_size; hd += 2) {
            float freq = 1.0f / powf(10000.0f, hd / (float)head_size);
            float val = pos * freq;
            table[((size_t)pos * head_size + hd)] = cosf(val);
            table[((size_t)pos * head_size + hd) + 1] = sinf(val);
        }
}

/* ------------------------------------------------------------------------ */

typedef struct {
    const uint8_t* q;
    const float* s;
} orc_qmat;

struct orc_model {
    int dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len, max_t;
    int wbits, group, kv_dim, head_size;
    const float* emb;
    const float* rms_att;
    const float* rms_ffn;
    const float* rms_final;
    orc_qmat wq, wk, wv, wo, w1, w2, w3, wcls;
    float *x, *xb, *xb2, *hb, *hb2, *q, *att, *logits, *kcache, *vcache;
    int kv8;                          /* 1: int8 KV cache (orc_model_set_kv8) */
    int kv8_splits;                   /* > 0: its attention in the split order (orc_model_set_kv8_splits) */
    int kv8_split_from;               /*      over more than this many positions */
    int8_t *k8, *v8;                  /* [L][max_t][kv_dim] */
    float *ks, *vs;                   /* [L][max_t][n_kv_heads] */
    int8_t* xq;
    float *xs, *xt;
};

static size_t qbytes(const orc_model* m, size_t rows, size_t cols) {
    return m->wbits == 4 ? rows * cols / 2 : rows * cols;
}

/* Tensor walk of runq.c:230-253. */
orc_model* orc_model_create(const int cfg[7], const void* weights, size_t bytes, int wbits,
                            int group, int max_t) {
    orc_model* m = (orc_model*)calloc(1, sizeof(*m));
    m->dim = cfg[0]; m->hidden = cfg[1]; m->n_layers = cfg[2]; m->n_heads = cfg[3];
    m->n_kv_heads = cfg[4]; m->vocab = cfg[5]; m->seq_len = cfg[6];
    m->max_t = (max_t > 0 && max_t < m->seq_len) ? max_t : m->seq_len;
    m->wbits = wbits; m->group = group;
    m->head_size = m->dim / m->n_heads;
    m->kv_dim = m->dim * m->n_kv_heads / m->n_heads;
    const size_t d = m->dim, h = m->hidden, L = m->n_layers, kv = m->kv_dim, V = m->vocab;
    const uint8_t* p = (const uint8_t*)weights;
    const uint8_t* end = p + bytes;
#define TAKEF(dst, n) do { dst = (const float*)p; p += (size_t)(n) * 4; } while (0)
#define TAKEQ(dst, rows, cols) do { dst.q = p; p += qbytes(m, rows, cols); \
        dst.s = (const float*)p; p += (size_t)(rows) * ((cols) / group) * 4; } while (0)
    TAKEF(m->emb, V * d);
    TAKEF(m->rms_att, L * d);
    TAKEQ(m->wq, L * d, d);
    TAKEQ(m->wk, L * kv, d);
    TAKEQ(m->wv, L * kv, d);
    TAKEQ(m->wo, L * d, d);
    TAKEF(m->rms_ffn, L * d);
    TAKEQ(m->w1, L * h, d);
    TAKEQ(m->w2, L * d, h);
    TAKEQ(m->w3, L * h, d);
    TAKEF(m->rms_final, d);
    TAKEQ(m->wcls, V, d);
#undef TAKEF
#undef TAKEQ
    if (p > end) { free(m); return NULL; }
    size_t maxn = h > d ? h : d;
    m->x = calloc(d, 4); m->xb = calloc(d, 4); m->xb2 = calloc(d, 4);
    m->hb = calloc(h, 4); m->hb2 = calloc(h, 4); m->q = calloc(d, 4);
    m->att = calloc((size_t)m->n_heads * m->max_t, 4);
    m->logits = calloc(V, 4);
    m->kcache = calloc(L * (size_t)m->max_t * kv, 4);
    m->vcache = calloc(L * (size_t)m->max_t * kv, 4);
    m->xq = calloc(maxn, 1);
    m->xs = calloc(maxn / group, 4);
    m->xt = calloc(maxn / group, 4);
    if (!m->kcache || !m->vcache) { orc_model_free(m); return NULL; }
    return m;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2); free(m->q);
    free(m->att); free(m->logits); free(m->kcache); free(m->vcache);
    free(m->k8); free(m->v8); free(m->ks); free(m->vs);
    free(m->xq); free(m->xs); free(m->xt);
    free(m);
}

static void matmul(orc_model* m, float* out, orc_qmat w, int layer, int rows, int cols) {
    const size_t nb = cols / m->group;
    const uint8_t* q = w.q + (size_t)layer * rows * (m->wbits == 4 ? cols / 2 : cols);
    const float* s = w.s + (size_t)layer * rows * nb;
    if (m->wbits == 4) orc_matmul_q4(out, m->xq, m->xs, m->xt, q, s, rows, cols, m->group, NULL);
    else orc_matmul_q8(out, m->xq, m->xs, m->xt, q, s, rows, cols, m->group, NULL);
}

/* runq.c:376-378, `score += q[i] * k[i]`, as the GCC -O3 -march=native
 * build evaluates it: the vectorised part (whole blocks of 8) multiplies
 * without fusing and adds the products in order; the scalar remainder
 * is contracted into FMAs. */
static float attn_score(const float* q, const float* k, int hs) {
    float score = 0.0f;
    const int nv = hs & ~7;
    int i = 0;
    for (; i < nv; i++) score = score + q[i] * k[i];
    for (; i < hs; i++) score = fmaf(q[i], k[i], score);
    return score;
}

/* RoPE, runq.c:351-365: rotate pairs of q over dim and of k over kv_dim.
 * GCC -O3 -march=native evaluates each rotation as
 * v0' = fma(v0, c, -(v1*s)) and v1' = fma(v0, s, v1*c). */
void orc_rope(float* q, float* k, int pos, int dim, int kv_dim, int hs) {
    for (int i = 0; i < dim; i += 2) {
        int head_dim = i % hs;
        float freq = 1.0f / powf(10000.0f, head_dim / (float)hs);
        float val = pos * freq;
        float fcr = cosf(val), fci = sinf(val);
        int rotn = i < kv_dim ? 2 : 1;
        for (int r = 0; r < rotn; r++) {
            float* vec = r == 0 ? q : k;
            float v0 = vec[i], v1 = vec[i + 1];
            vec[i] = fmaf(v0, fcr, -(v1 * fci));
            vec[i + 1] = fmaf(v0, fci, v1 * fcr);
        }
    }
}

/* Multi-head attention of runq.c:367-391 (+ softmax :307-318) for one
 * layer.  Position t of kv head g is at kc + g*head_stride + t*t_stride. */
void orc_attention(const float* q, const float* kc, const float* vc, float* out, int pos,
                   int n_heads, int n_kv_heads, int hs, size_t t_stride, size_t head_stride,
                   float* att_scratch, int att_stride) {
    const int kv_mul = n_heads / n_kv_heads;
    const float rs = sqrtf((float)hs);
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const float* qh = q + (size_t)h * hs;
        float* att = att_scratch + (size_t)h * att_stride;
        const size_t hoff = (size_t)(h / kv_mul) * head_stride;
        for (int t = 0; t <= pos; t++) att[t] = attn_score(qh, kc + hoff + (size_t)t * t_stride, hs) / rs;
        orc_softmax(att, pos + 1);
        float* xb = out + (size_t)h * hs;
        memset(xb, 0, hs * sizeof(float));
        for (int t = 0; t <= pos; t++) {
            const float* vt = vc + hoff + (size_t)t * t_stride;
            float a = att[t];
            for (int i = 0; i < hs; i++) xb[i] = fmaf(a, vt[i], xb[i]);
        }
    }
}

/* One kv head's row of the int8 KV cache, v5-cuda-fused/run.cu:204-249
 * (kv_quant_kernel): amax over the row, s = amax/127 (1e-8 when 0),
 * q = clamp(rint(v/s), -127, 127) (__float2int_rn of the quotient). */
void orc_kv_quant(const float* row, int hs, int8_t* q, float* s) {
    float amax = 0.0f;
    for (int i = 0; i < hs; i++) { float a = fabsf(row[i]); if (a > amax) amax = a; }
    float sc = amax / 127.0f;
    if (sc == 0.0f) sc = 1e-8f;
    for (int i = 0; i < hs; i++) {
        float r = rintf(row[i] / sc);
        r = r > 127.0f ? 127.0f : (r < -127.0f ? -127.0f : r);
        q[i] = (int8_t)r;
    }
    *s = sc;
}

/* Attention over the int8 cache, v5-cuda-fused/run.cu:350-410
 * (attention_cache_kernel): score_t = (q . k8_t) / sqrt(hs) * ks_t,
 * softmax over t <= pos, out = sum_t p_t * vs_t * v8_t.  Evaluated in double
 * (the reference's float order is a warp reduction; this is the value every
 * order approximates).  Row t of kv head g: kc + g*head_stride + t*t_stride;
 * its scale: ks[t*s_t_stride + g*s_head_stride]. */
void orc_attention_kv8(const float* q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
                       float* out, int pos, int n_heads, int n_kv_heads, int hs, size_t t_stride,
                       size_t head_stride, size_t s_t_stride, size_t s_head_stride) {
    const int kv_mul = n_heads / n_kv_heads;
    const double rs = sqrt((double)hs);
    double* sc = (double*)malloc((size_t)(pos + 1) * sizeof(double));
    double* acc = (double*)malloc((size_t)hs * sizeof(double));
    for (int h = 0; h < n_heads; h++) {
        const int g = h / kv_mul;
        const float* qh = q + (size_t)h * hs;
        double m = -INFINITY;
        for (int t = 0; t <= pos; t++) {
            const int8_t* kt = kc + (size_t)g * head_stride + (size_t)t * t_stride;
            double d = 0.0;
            for (int i = 0; i < hs; i++) d += (double)qh[i] * (double)kt[i];
            sc[t] = d / rs * (double)ks[(size_t)t * s_t_stride + (size_t)g * s_head_stride];
            if (sc[t] > m) m = sc[t];
        }
        double sum = 0.0;
        for (int t = 0; t <= pos; t++) { sc[t] = exp(sc[t] - m); sum += sc[t]; }
        for (int i = 0; i < hs; i++) acc[i] = 0.0;
        for (int t = 0; t <= pos; t++) {
            const int8_t* vt = vc + (size_t)g * head_stride + (size_t)t * t_stride;
            const double w = sc[t] * (double)vs[(size_t)t * s_t_stride + (size_t)g * s_head_stride];
            for (int i = 0; i < hs; i++) acc[i] += w * (double)vt[i];
        }
        for (int i = 0; i < hs; i++) out[(size_t)h * hs + i] = (float)(acc[i] / sum);
    }
    free(sc);
    free(acc);
}

/* The same attention in the float order of this build's GPU kernels
 * (k_attn8_fused), so that the int8-KV decode can be
 * compared bit for bit; pinned to orc_attention_kv8 (double) by the tests.
 *   score_t: four partial FMA chains, chain j over the 4-element chunks
 *            c = 4j + 16i in order, combined as (a0+a1)+(a2+a3); then
 *            (dot / sqrtf(hs)) * ks_t
 *   sum:     1024 partial sums (thread j: t = j, j+1024, ...), each wave's 64
 *            combined by the xor butterfly 32,16,...,1, the 16 waves by a
 *            pairwise tree ((w0+w1)+(w2+w3))+...; e_t = expf(score_t - max)
 *   out[d]:  S = 1024/(hs/4) slices, slice s: fma(e_t*vs_t, v8_t[d], acc)
 *            over t = s, s+S, ...; out = (((0+p_0)+p_1)+...+p_{S-1}) / sum */
static float butterfly64(float* v) {
    for (int o = 32; o > 0; o >>= 1) {
        float w[64];
        for (int l = 0; l < 64; l++) w[l] = v[l] + v[l ^ o];
        memcpy(v, w, sizeof w);
    }
    return v[0];
}

void orc_attention_kv8_ordered(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                               const float* vs, float* out, int pos, int n_heads, int n_kv_heads, int hs,
                               size_t t_stride, size_t head_stride, size_t s_t_stride, size_t s_head_stride) {
    const int kv_mul = n_heads / n_kv_heads, n = pos + 1;
    const float rs = sqrtf((float)hs);
    float* sc = (float*)malloc((size_t)n * sizeof(float));
    float* pe = (float*)malloc((size_t)n * sizeof(float));
    for (int h = 0; h < n_heads; h++) {
        const int g = h / kv_mul;
        const float* qh = q + (size_t)h * hs;
        float m = -INFINITY;
        for (int t = 0; t < n; t++) {
            const int8_t* kt = kc + (size_t)g * head_stride + (size_t)t * t_stride;
            float a[4];
            for (int j = 0; j < 4; j++) {
                a[j] = 0.0f;
                for (int c = 4 * j; c < hs; c += 16)
                    for (int e = 0; e < 4; e++) a[j] = fmaf(qh[c + e], (float)kt[c + e], a[j]);
            }
            const float dot = (a[0] + a[1]) + (a[2] + a[3]);
            sc[t] = dot / rs * ks[(size_t)t * s_t_stride + (size_t)g * s_head_stride];
            m = fmaxf(m, sc[t]);
        }
        float part[1024], wsum[16];
        for (int j = 0; j < 1024; j++) {
            part[j] = 0.0f;
            for (int t = j; t < n; t += 1024) {
                const float e = expf(sc[t] - m);
                part[j] = part[j] + e;
                pe[t] = e * vs[(size_t)t * s_t_stride + (size_t)g * s_head_stride];
            }
        }
        for (int w = 0; w < 16; w++) wsum[w] = butterfly64(part + 64 * w);
        for (int width = 8; width >= 1; width /= 2)
            for (int w = 0; w < width; w++) wsum[w] = wsum[2 * w] + wsum[2 * w + 1];
        const float sum = wsum[0];
        const int groups = hs / 4, slices = 1024 / groups;
        for (int d = 0; d < hs; d++) {
            float s = 0.0f;
            for (int sl = 0; sl < slices; sl++) {
                float acc = 0.0f;
                for (int t = sl; t < n; t += slices)
                    acc = fmaf(pe[t], (float)vc[(size_t)g * head_stride + (size_t)t * t_stride + d], acc);
                s = s + acc;
            }
            out[(size_t)h * hs + d] = s / sum;
        }
    }
    free(sc);
    free(pe);
}

/* The int8-KV attention split over the context (the float order of this
 * build's k_attn8_split, for bit-exact comparison; pinned to
 * orc_attention_kv8 (double) by the tests).  n = pos + 1 positions in S
 * splits of C = ceil(n / S): split s covers [min(sC, n), min(n, sC + C)).
 * Per split:
 *   score_t  as orc_attention_kv8_ordered: four FMA chains (chain j over the
 *            4-element chunks c = 4j + 16i), (a0+a1)+(a2+a3), then
 *            (dot / sqrtf(hs)) * ks_t
 *   m_s      the split's maximum score; e_t = expf(score_t - m_s)
 *   l_s      256 partial sums (thread j: t = t0 + j, t0 + j + 256, ...; at
 *            most one position each since C <= 256), the 4 waves' 64 added by
 *            the xor butterfly 32,16,...,1, the waves as (w0+w1)+(w2+w3)
 *   o_s[d]   slices = 256/(hs/4); slice k: fma(e_t*vs_t, v8_t[d], acc) over
 *            t = t0 + k, t0 + k + slices, ...; o = ((0+p_0)+p_1)+...
 * Merge in split order: M = max m_s, w_s = expf(m_s - M) (0 for an empty
 * split), L = ((0 + w_0*l_0) + w_1*l_1) + ..., out[d] = acc / L with
 * acc = fmaf(w_s, o_s[d], acc) over s. */
void orc_attention_kv8_split(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                             const float* vs, float* out, int pos, int n_heads, int n_kv_heads, int hs,
                             size_t t_stride, size_t head_stride, size_t s_t_stride, size_t s_head_stride,
                             int S) {
    const int kv_mul = n_heads / n_kv_heads, n = pos + 1, C = (n + S - 1) / S;
    if (S < 1 || C > 256) {
        fprintf(stderr, "orc_attention_kv8_split: %d positions in %d splits exceed 256 per split\n", n, S);
        abort();
    }
    const float rs = sqrtf((float)hs);
    float* pm = (float*)malloc((size_t)S * sizeof(float));
    float* pl = (float*)malloc((size_t)S * sizeof(float));
    float* po = (float*)malloc((size_t)S * hs * sizeof(float));
    float sc[256], pe[256];
    for (int h = 0; h < n_heads; h++) {
        const int g = h / kv_mul;
        const float* qh = q + (size_t)h * hs;
        for (int sp = 0; sp < S; sp++) {
            const int t0 = sp * C < n ? sp * C : n;
            const int t1 = t0 + C < n ? t0 + C : n, mn = t1 - t0;
            float m = -INFINITY;
            for (int t = t0; t < t1; t++) {
                const int8_t* kt = kc + (size_t)g * head_stride + (size_t)t * t_stride;
                float a[4];
                for (int j = 0; j < 4; j++) {
                    a[j] = 0.0f;
                    for (int c = 4 * j; c < hs; c += 16)
                        for (int e = 0; e < 4; e++) a[j] = fmaf(qh[c + e], (float)kt[c + e], a[j]);
                }
                const float dot = (a[0] + a[1]) + (a[2] + a[3]);
                sc[t - t0] = dot / rs * ks[(size_t)t * s_t_stride + (size_t)g * s_head_stride];
                m = fmaxf(m, sc[t - t0]);
            }
            float part[256], wsum[4];
            for (int j = 0; j < 256; j++) {
                part[j] = 0.0f;
                if (j < mn) {
                    const int t = t0 + j;
                    const float e = expf(sc[j] - m);
                    part[j] = part[j] + e;
                    pe[j] = e * vs[(size_t)t * s_t_stride + (size_t)g * s_head_stride];
                }
            }
            for (int w = 0; w < 4; w++) wsum[w] = butterfly64(part + 64 * w);
            pm[sp] = mn > 0 ? m : -INFINITY;
            pl[sp] = mn > 0 ? (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]) : 0.0f;
            const int slices = 256 / (hs / 4);
            for (int d = 0; d < hs; d++) {
                float o = 0.0f;
                for (int k = 0; k < slices; k++) {
                    float acc = 0.0f;
                    for (int j = k; j < mn; j += slices)
                        acc = fmaf(pe[j], (float)vc[(size_t)g * head_stride + (size_t)(t0 + j) * t_stride + d], acc);
                    o = o + acc;
                }
                po[(size_t)sp * hs + d] = o;
            }
        }
        float M = -INFINITY;
        for (int sp = 0; sp < S; sp++) M = fmaxf(M, pm[sp]);
        float L = 0.0f;
        for (int sp = 0; sp < S; sp++) {
            const float w = pm[sp] == -INFINITY ? 0.0f : expf(pm[sp] - M);
            pm[sp] = w;
            L = L + w * pl[sp];
        }
        for (int d = 0; d < hs; d++) {
            float acc = 0.0f;
            for (int sp = 0; sp < S; sp++) acc = fmaf(pm[sp], po[(size_t)sp * hs + d], acc);
            out[(size_t)h * hs + d] = acc / L;
        }
    }
    free(pm);
    free(pl);
    free(po);
}

int orc_model_set_kv8_splits(orc_model* m, int splits, int split_from) {
    if (splits < 0 || splits > 64 || split_from < 0) return -1;
    m->kv8_splits = splits;
    m->kv8_split_from = split_from;
    return 0;
}

int orc_model_set_kv8(orc_model* m, int on) {
    if (!on) { m->kv8 = 0; return 0; }
    const size_t n = (size_t)m->n_layers * m->max_t * m->kv_dim;
    const size_t ns = (size_t)m->n_layers * m->max_t * m->n_kv_heads;
    if (!m->k8) {
        m->k8 = calloc(n, 1); m->v8 = calloc(n, 1);
        m->ks = calloc(ns, 4); m->vs = calloc(ns, 4);
        if (!m->k8 || !m->v8 || !m->ks || !m->vs) return -1;
    }
    m->kv8 = 1;
    return 0;
}

/* SwiGLU, runq.c:405-410: out = (h * (1/(1+expf(-h)))) * h2. */
void orc_swiglu(float* out, const float* h, const float* h2, int n) {
    for (int i = 0; i < n; i++) {
        float val = h[i];
        val *= (1.0f / (1.0f + expf(-val)));
        val *= h2[i];
        out[i] = val;
    }
}

/* runq.c:320-421 with the group size and weight width as parameters. */
const float* orc_forward(orc_model* m, int token, int pos, float* x_layers) {
    const int dim = m->dim, kv_dim = m->kv_dim, hs = m->head_size, hidden = m->hidden;
    const int G = m->group;
    float* x = m->x;
    memcpy(x, m->emb + (size_t)token * dim, dim * sizeof(float));
    if (x_layers) memcpy(x_layers, x, dim * sizeof(float));

    for (int l = 0; l < m->n_layers; l++) {
        orc_rmsnorm(m->xb, x, m->rms_att + (size_t)l * dim, dim);
        size_t loff = (size_t)l * m->max_t * kv_dim;
        float* k = m->kcache + loff + (size_t)pos * kv_dim;
        float* v = m->vcache + loff + (size_t)pos * kv_dim;
        orc_quantize_act(m->xb, dim, G, m->xq, m->xs, m->xt);
        matmul(m, m->q, m->wq, l, dim, dim);
        matmul(m, k, m->wk, l, kv_dim, dim);
        matmul(m, v, m->wv, l, kv_dim, dim);

        orc_rope(m->q, k, pos, dim, kv_dim, hs);

        if (m->kv8) {
            /* v5-cuda-fused/run.cu:627-631: the rotated k and the v row of
             * this position go into the int8 cache, one scale per kv head */
            const size_t soff = (size_t)l * m->max_t * m->n_kv_heads + (size_t)pos * m->n_kv_heads;
            for (int g = 0; g < m->n_kv_heads; g++) {
                orc_kv_quant(k + (size_t)g * hs, hs, m->k8 + loff + (size_t)pos * kv_dim + (size_t)g * hs, m->ks + soff + g);
                orc_kv_quant(v + (size_t)g * hs, hs, m->v8 + loff + (size_t)pos * kv_dim + (size_t)g * hs, m->vs + soff + g);
            }
            const size_t sl = (size_t)l * m->max_t * m->n_kv_heads;
            if (m->kv8_splits > 0 && pos + 1 > m->kv8_split_from)
                orc_attention_kv8_split(m->q, m->k8 + loff, m->v8 + loff, m->ks + sl, m->vs + sl, m->xb, pos,
                                        m->n_heads, m->n_kv_heads, hs, (size_t)kv_dim, (size_t)hs,
                                        (size_t)m->n_kv_heads, 1, m->kv8_splits);
            else
                orc_attention_kv8_ordered(m->q, m->k8 + loff, m->v8 + loff, m->ks + sl, m->vs + sl, m->xb, pos,
                                          m->n_heads, m->n_kv_heads, hs, (size_t)kv_dim, (size_t)hs,
                                          (size_t)m->n_kv_heads, 1);
        } else {
            orc_attention(m->q, m->kcache + loff, m->vcache + loff, m->xb, pos, m->n_heads,
                          m->n_kv_heads, hs, (size_t)kv_dim, (size_t)hs, m->att, m->max_t);
        }

        orc_quantize_act(m->xb, dim, G, m->xq, m->xs, m->xt);
        matmul(m, m->xb2, m->wo, l, dim, dim);
        for (int i = 0; i < dim; i++) x[i] += m->xb2[i];

        orc_rmsnorm(m->xb, x, m->rms_ffn + (size_t)l * dim, dim);
        orc_quantize_act(m->xb, dim, G, m->xq, m->xs, m->xt);
        matmul(m, m->hb, m->w1, l, hidden, dim);
        matmul(m, m->hb2, m->w3, l, hidden, dim);
        orc_swiglu(m->hb, m->hb, m->hb2, hidden);
        orc_quantize_act(m->hb, hidden, G, m->xq, m->xs, m->xt);
        matmul(m, m->xb, m->w2, l, dim, hidden);
        for (int i = 0; i < dim; i++) x[i] += m->xb[i];
        if (x_layers) memcpy(x_layers + (size_t)(l + 1) * dim, x, dim * sizeof(float));
    }

    orc_rmsnorm(x, x, m->rms_final, dim);
    orc_quantize_act(x, dim, G, m->xq, m->xs, m->xt);
    if (m->wbits == 4)
        orc_matmul_q4(m->logits, m->xq, m->xs, m->xt, m->wcls.q, m->wcls.s, m->vocab, dim, G, NULL);
    else
        orc_matmul_q8(m->logits, m->xq, m->xs, m->xt, m->wcls.q, m->wcls.s, m->vocab, dim, G, NULL);
    return m->logits;
}

void orc_greedy(orc_model* m, const int* prompt, int n_prompt, int n_steps, int* ids_out) {
    int token = prompt[0];
    for (int pos = 0; pos < n_steps; pos++) {
        const float* logits = orc_forward(m, token, pos, NULL);
        int next = pos < n_prompt - 1 ? prompt[pos + 1] : orc_argmax(logits, m->vocab);
        ids_out[pos] = next;
        token = next;
    }
}

/* glibc expf over an array (the host function the reference calls). */
void orc_expf_array(const float* x, float* y, size_t n) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) y[i] = expf(x[i]);
}
