// engine.hip - the decode engine behind l2q_engine_* (include/l2q.h).
//
// Device layout (one weight arena, one state arena, both hipMalloc'd once):
//   emb        fp32 [V][d]            rms_att / rms_ffn fp32 [L][d], rms_final [d]
//   qkv_w      [L][d + 2kv][d*bits/8] rows of wq, wk, wv of a layer, back to back
//   qkv_s      [L][d + 2kv][d/G]      fp32 scales in the same row order
//   wo_w/s     [L][d][...]            as in the file
//   w13_w/s    [L][2h][...]           rows of w1 then w3 of a layer
//   w2_w/s     [L][d][...]
//   wcls_w/s   [V][...]
//   INT8 weights are stored signed (the file's +128 bias removed at load).
//   kcache/vcache fp32 [L][n_kv_heads][max_t][hs]
// Concatenating wq|wk|wv and w1|w3 turns 5 GEMV launches per layer into 2
// with 12288- and 22016-row grids at the 7B shape.
//
// One decode step (runq.c:320-421) is captured once into a hipGraph; the
// token and position are read from device memory (`meta`), so every step
// replays the same graph after an 8-byte upload (as v5-cuda-fused/run.cu:
// 671-695 does).
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include <new>
#include <vector>

#include "launch.h"
#include "qformat.h"

struct l2q_engine {
    l2q_config cfg;
    int wbits, G, max_t, kv_dim, hs, S;
    int device;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr, graph_am = nullptr;
    hipGraphExec_t exec = nullptr, exec_am = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    char* warena = nullptr;
    char* sarena = nullptr;
    size_t wbytes = 0, sbytes = 0;
    // weights
    float *emb, *rms_att, *rms_ffn, *rms_final;
    uint8_t *qkv_w, *wo_w, *w13_w, *w2_w, *wcls_w;
    float *qkv_s, *wo_s, *w13_s, *w2_s, *wcls_s;
    size_t rowb_d, rowb_h;   // weight bytes of a row with d / h columns
    // state
    float *x, *qkv, *att, *wo_out, *h13, *ffn_out, *logits;
    int8_t* xq;
    float* xs;
    float *kcache, *vcache, *rope, *scores;
    int *meta, *am;
    int* h_meta = nullptr;   // pinned {token, pos} slots
    int h_meta_slots = 0;
    int* h_am = nullptr;     // pinned argmax result
};

using namespace l2q;

namespace {

#define HIPCHK(call, what)                            \
    do {                                              \
        hipError_t e_ = (call);                       \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Arena {
    size_t used = 0;
    size_t take(size_t bytes) {
        size_t o = align_up(used, 256);
        used = o + bytes;
        return o;
    }
};

// Enqueue one decode step on `st` (captured or eager).  If `dbg_x` is set
// (eager diagnostic mode) the residual stream after the embedding and after
// each layer is copied to it.
int enqueue_step(l2q_engine* e, hipStream_t st, float* dbg_x, float* dbg_tmp, bool argmax) {
    const l2q_config& c = e->cfg;
    const int d = c.dim, h = c.hidden_dim, kv = e->kv_dim, G = e->G, bits = e->wbits;
    const int qkv_rows = d + 2 * kv;
    const size_t nbd = (size_t)d / G, nbh = (size_t)h / G;
    int rc;
    for (int l = 0; l < c.n_layers; l++) {
        // attention rmsnorm; the FFN output of layer l-1 is the pending residual
        rc = launch_rmsnorm_quant(e->x, l == 0 ? e->emb : nullptr, e->meta, l == 0 ? nullptr : e->ffn_out, e->x,
                                  e->rms_att + (size_t)l * d, d, G, e->xq, e->xs, st);
        if (rc) return rc;
        if (dbg_x && l == 0) HIPCHK(hipMemcpyAsync(dbg_x, e->x, d * sizeof(float), hipMemcpyDeviceToHost, st), "copy x");
        GemvArgs qa{e->qkv, e->xq, e->xs, e->qkv_w + (size_t)l * qkv_rows * e->rowb_d,
                    e->qkv_s + (size_t)l * qkv_rows * nbd, qkv_rows, d, nullptr};
        if ((rc = launch_gemv(bits, G, qa, st))) return rc;
        float* kc = e->kcache + (size_t)l * kv * e->max_t;
        float* vc = e->vcache + (size_t)l * kv * e->max_t;
        rc = launch_rope_kv_append(e->qkv, e->qkv + d, e->qkv + d + kv, kc, vc, e->rope, e->meta, 0, d, kv, e->hs,
                                   e->max_t, st);
        if (rc) return rc;
        rc = launch_attention_exact(e->qkv, kc, vc, e->att, e->scores, e->S, e->meta, 0, c.n_heads, c.n_kv_heads,
                                    e->hs, e->max_t, st);
        if (rc) return rc;
        if ((rc = launch_quantize(e->att, d, G, e->xq, e->xs, st))) return rc;
        GemvArgs oa{e->wo_out, e->xq, e->xs, e->wo_w + (size_t)l * d * e->rowb_d, e->wo_s + (size_t)l * d * nbd, d, d,
                    nullptr};
        if ((rc = launch_gemv(bits, G, oa, st))) return rc;
        // ffn rmsnorm; the attention output is the pending residual (persisted into x)
        rc = launch_rmsnorm_quant(e->x, nullptr, e->meta, e->wo_out, e->x, e->rms_ffn + (size_t)l * d, d, G, e->xq,
                                  e->xs, st);
        if (rc) return rc;
        GemvArgs ha{e->h13, e->xq, e->xs, e->w13_w + (size_t)l * 2 * h * e->rowb_d,
                    e->w13_s + (size_t)l * 2 * h * nbd, 2 * h, d, nullptr};
        if ((rc = launch_gemv(bits, G, ha, st))) return rc;
        if ((rc = launch_swiglu_quant(e->h13, e->h13 + h, h, G, e->xq, e->xs, nullptr, st))) return rc;
        GemvArgs fa{e->ffn_out, e->xq, e->xs, e->w2_w + (size_t)l * d * e->rowb_h, e->w2_s + (size_t)l * d * nbh, d, h,
                    nullptr};
        if ((rc = launch_gemv(bits, G, fa, st))) return rc;
        if (dbg_x) {
            float* dst = dbg_x + (size_t)(l + 1) * d;
            HIPCHK(hipMemcpyAsync(dst, e->x, d * sizeof(float), hipMemcpyDeviceToHost, st), "copy x");
            HIPCHK(hipMemcpyAsync(dbg_tmp, e->ffn_out, d * sizeof(float), hipMemcpyDeviceToHost, st), "copy ffn");
            HIPCHK(hipStreamSynchronize(st), "sync");
            for (int i = 0; i < d; i++) dst[i] = dst[i] + dbg_tmp[i];   // the add the next norm performs
        }
    }
    rc = launch_rmsnorm_quant(e->x, nullptr, e->meta, e->ffn_out, e->x, e->rms_final, d, G, e->xq, e->xs, st);
    if (rc) return rc;
    GemvArgs ca{e->logits, e->xq, e->xs, e->wcls_w, e->wcls_s, c.vocab_size, d, nullptr};
    if ((rc = launch_gemv(bits, G, ca, st))) return rc;
    if (argmax) return launch_argmax(e->logits, c.vocab_size, e->am, st);
    return L2Q_OK;
}

int capture(l2q_engine* e, bool argmax, hipGraph_t* g, hipGraphExec_t* ex) {
    HIPCHK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    int rc = enqueue_step(e, e->stream, nullptr, nullptr, argmax);
    hipGraph_t graph = nullptr;
    hipError_t ee = hipStreamEndCapture(e->stream, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (ee != hipSuccess) return hip_fail(ee, "hipStreamEndCapture");
    *g = graph;
    HIPCHK(hipGraphInstantiate(ex, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    return L2Q_OK;
}

void release(l2q_engine* e) {
    if (e->exec) (void)hipGraphExecDestroy(e->exec);
    if (e->exec_am) (void)hipGraphExecDestroy(e->exec_am);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    if (e->graph_am) (void)hipGraphDestroy(e->graph_am);
    if (e->ev0) (void)hipEventDestroy(e->ev0);
    if (e->ev1) (void)hipEventDestroy(e->ev1);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    if (e->warena) (void)hipFree(e->warena);
    if (e->sarena) (void)hipFree(e->sarena);
    if (e->h_meta) (void)hipHostFree(e->h_meta);
    if (e->h_am) (void)hipHostFree(e->h_am);
}

int copy_h2d(void* dst, const void* src, size_t n) {
    HIPCHK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice), "hipMemcpy(weights)");
    return L2Q_OK;
}

int build(l2q_engine* e, const void* weights, size_t weights_bytes) {
    const l2q_config& c = e->cfg;
    const size_t d = c.dim, h = c.hidden_dim, L = c.n_layers, V = c.vocab_size, kv = e->kv_dim;
    const int bits = e->wbits, G = e->G;
    qll_layout lay;
    if (qll_layout_compute(&c, bits, G, &lay)) { set_error("engine: inconsistent config"); return L2Q_ERR_ARG; }
    if (weights_bytes < lay.total) {
        set_error("engine: weights image has %zu bytes, config needs %zu", weights_bytes, lay.total);
        return L2Q_ERR_FORMAT;
    }
    e->rowb_d = qll_matrix_bytes(1, d, bits);
    e->rowb_h = qll_matrix_bytes(1, h, bits);
    const size_t nbd = d / G, nbh = h / G;
    const size_t qkv_rows = d + 2 * kv;

    // weight arena: all quantized weight bytes first (one un-bias pass for INT8)
    Arena wa;
    const size_t o_qkv_w = wa.take(L * qkv_rows * e->rowb_d);
    const size_t o_wo_w = wa.take(L * d * e->rowb_d);
    const size_t o_w13_w = wa.take(L * 2 * h * e->rowb_d);
    const size_t o_w2_w = wa.take(L * d * e->rowb_h);
    const size_t o_wcls_w = wa.take(V * e->rowb_d);
    const size_t qbytes_end = wa.used;
    const size_t o_qkv_s = wa.take(L * qkv_rows * nbd * 4);
    const size_t o_wo_s = wa.take(L * d * nbd * 4);
    const size_t o_w13_s = wa.take(L * 2 * h * nbd * 4);
    const size_t o_w2_s = wa.take(L * d * nbh * 4);
    const size_t o_wcls_s = wa.take(V * nbd * 4);
    const size_t o_emb = wa.take(V * d * 4);
    const size_t o_ra = wa.take(L * d * 4);
    const size_t o_rf = wa.take(L * d * 4);
    const size_t o_rl = wa.take(d * 4);
    e->wbytes = align_up(wa.used, 256);
    HIPCHK(hipMalloc(&e->warena, e->wbytes), "hipMalloc(weights)");
    char* W = e->warena;
    e->qkv_w = (uint8_t*)(W + o_qkv_w); e->wo_w = (uint8_t*)(W + o_wo_w); e->w13_w = (uint8_t*)(W + o_w13_w);
    e->w2_w = (uint8_t*)(W + o_w2_w); e->wcls_w = (uint8_t*)(W + o_wcls_w);
    e->qkv_s = (float*)(W + o_qkv_s); e->wo_s = (float*)(W + o_wo_s); e->w13_s = (float*)(W + o_w13_s);
    e->w2_s = (float*)(W + o_w2_s); e->wcls_s = (float*)(W + o_wcls_s);
    e->emb = (float*)(W + o_emb); e->rms_att = (float*)(W + o_ra); e->rms_ffn = (float*)(W + o_rf);
    e->rms_final = (float*)(W + o_rl);

    const uint8_t* F = (const uint8_t*)weights;
    int rc;
    if ((rc = copy_h2d(e->emb, F + lay.emb, V * d * 4))) return rc;
    if ((rc = copy_h2d(e->rms_att, F + lay.rms_att, L * d * 4))) return rc;
    if ((rc = copy_h2d(e->rms_ffn, F + lay.rms_ffn, L * d * 4))) return rc;
    if ((rc = copy_h2d(e->rms_final, F + lay.rms_final, d * 4))) return rc;
    for (size_t l = 0; l < L; l++) {
        uint8_t* qw = e->qkv_w + l * qkv_rows * e->rowb_d;
        float* qs = e->qkv_s + l * qkv_rows * nbd;
        if ((rc = copy_h2d(qw, F + lay.wq + l * d * e->rowb_d, d * e->rowb_d))) return rc;
        if ((rc = copy_h2d(qw + d * e->rowb_d, F + lay.wk + l * kv * e->rowb_d, kv * e->rowb_d))) return rc;
        if ((rc = copy_h2d(qw + (d + kv) * e->rowb_d, F + lay.wv + l * kv * e->rowb_d, kv * e->rowb_d))) return rc;
        if ((rc = copy_h2d(qs, F + lay.wq_s + l * d * nbd * 4, d * nbd * 4))) return rc;
        if ((rc = copy_h2d(qs + d * nbd, F + lay.wk_s + l * kv * nbd * 4, kv * nbd * 4))) return rc;
        if ((rc = copy_h2d(qs + (d + kv) * nbd, F + lay.wv_s + l * kv * nbd * 4, kv * nbd * 4))) return rc;
        uint8_t* hw = e->w13_w + l * 2 * h * e->rowb_d;
        float* hsc = e->w13_s + l * 2 * h * nbd;
        if ((rc = copy_h2d(hw, F + lay.w1 + l * h * e->rowb_d, h * e->rowb_d))) return rc;
        if ((rc = copy_h2d(hw + h * e->rowb_d, F + lay.w3 + l * h * e->rowb_d, h * e->rowb_d))) return rc;
        if ((rc = copy_h2d(hsc, F + lay.w1_s + l * h * nbd * 4, h * nbd * 4))) return rc;
        if ((rc = copy_h2d(hsc + h * nbd, F + lay.w3_s + l * h * nbd * 4, h * nbd * 4))) return rc;
    }
    if ((rc = copy_h2d(e->wo_w, F + lay.wo, L * d * e->rowb_d))) return rc;
    if ((rc = copy_h2d(e->wo_s, F + lay.wo_s, L * d * nbd * 4))) return rc;
    if ((rc = copy_h2d(e->w2_w, F + lay.w2, L * d * e->rowb_h))) return rc;
    if ((rc = copy_h2d(e->w2_s, F + lay.w2_s, L * d * nbh * 4))) return rc;
    if ((rc = copy_h2d(e->wcls_w, F + lay.wcls, V * e->rowb_d))) return rc;
    if ((rc = copy_h2d(e->wcls_s, F + lay.wcls_s, V * nbd * 4))) return rc;
    if (bits == 8) {
        if ((rc = launch_unbias((const uint8_t*)W, (int8_t*)W, qbytes_end, e->stream))) return rc;
    }

    // state arena
    Arena sa;
    const size_t maxn = h > d ? h : d;
    const size_t o_x = sa.take(d * 4), o_qkv = sa.take(qkv_rows * 4), o_att = sa.take(d * 4);
    const size_t o_wo = sa.take(d * 4), o_h13 = sa.take(2 * h * 4), o_ffn = sa.take(d * 4);
    const size_t o_logits = sa.take(V * 4), o_xq = sa.take(maxn), o_xs = sa.take(maxn / G * 4);
    const size_t kvfloats = L * kv * (size_t)e->max_t;
    const size_t o_kc = sa.take(kvfloats * 4), o_vc = sa.take(kvfloats * 4);
    const size_t o_rope = sa.take((size_t)e->max_t * e->hs * 4);
    const size_t o_sc = sa.take((size_t)c.n_heads * e->max_t * 4);
    const size_t o_meta = sa.take(2 * sizeof(int)), o_am = sa.take(sizeof(int));
    e->sbytes = align_up(sa.used, 256);
    HIPCHK(hipMalloc(&e->sarena, e->sbytes), "hipMalloc(state)");
    char* S_ = e->sarena;
    e->x = (float*)(S_ + o_x); e->qkv = (float*)(S_ + o_qkv); e->att = (float*)(S_ + o_att);
    e->wo_out = (float*)(S_ + o_wo); e->h13 = (float*)(S_ + o_h13); e->ffn_out = (float*)(S_ + o_ffn);
    e->logits = (float*)(S_ + o_logits); e->xq = (int8_t*)(S_ + o_xq); e->xs = (float*)(S_ + o_xs);
    e->kcache = (float*)(S_ + o_kc); e->vcache = (float*)(S_ + o_vc); e->rope = (float*)(S_ + o_rope);
    e->scores = (float*)(S_ + o_sc);
    e->meta = (int*)(S_ + o_meta); e->am = (int*)(S_ + o_am);
    // zero-fill the state (outside any graph) so unused cache rows are defined
    HIPCHK(hipMemsetAsync(e->sarena, 0, e->sbytes, e->stream), "hipMemset(state)");

    std::vector<float> rope((size_t)e->max_t * e->hs);
    l2q_rope_table(rope.data(), e->max_t, e->hs);
    HIPCHK(hipMemcpyAsync(e->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice, e->stream), "copy rope");
    HIPCHK(hipStreamSynchronize(e->stream), "sync(build)");

    e->h_meta_slots = 1;
    HIPCHK(hipHostMalloc((void**)&e->h_meta, 2 * sizeof(int) * e->h_meta_slots, hipHostMallocDefault), "hipHostMalloc");
    HIPCHK(hipHostMalloc((void**)&e->h_am, sizeof(int), hipHostMallocDefault), "hipHostMalloc");
    HIPCHK(hipEventCreate(&e->ev0), "hipEventCreate");
    HIPCHK(hipEventCreate(&e->ev1), "hipEventCreate");
    if ((rc = capture(e, false, &e->graph, &e->exec))) return rc;
    if ((rc = capture(e, true, &e->graph_am, &e->exec_am))) return rc;
    return L2Q_OK;
}

int check_step(l2q_engine* e, int token, int pos) {
    if (!e) { set_error("engine: null handle"); return L2Q_ERR_ARG; }
    if (token < 0 || token >= e->cfg.vocab_size) { set_error("engine: token %d out of range", token); return L2Q_ERR_ARG; }
    if (pos < 0 || pos >= e->max_t) {
        set_error("engine: position %d outside the KV cache (max_steps %d)", pos, e->max_t);
        return L2Q_ERR_STATE;
    }
    return L2Q_OK;
}

int launch_step(l2q_engine* e, int token, int pos, hipGraphExec_t ex, int slot) {
    int* hm = e->h_meta + 2 * slot;
    hm[0] = token;
    hm[1] = pos;
    HIPCHK(hipMemcpyAsync(e->meta, hm, 2 * sizeof(int), hipMemcpyHostToDevice, e->stream), "upload meta");
    HIPCHK(hipGraphLaunch(ex, e->stream), "hipGraphLaunch");
    return L2Q_OK;
}

}  // namespace

extern "C" {

int l2q_engine_create(const l2q_config* cfg, const void* weights, size_t weights_bytes, int wbits, int group,
                      int max_steps, l2q_engine** out) {
    if (!cfg || !weights || !out) { set_error("engine: null argument"); return L2Q_ERR_ARG; }
    *out = nullptr;
    const l2q_config& c = *cfg;
    if (c.dim <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.dim % c.n_heads || c.n_heads % c.n_kv_heads) {
        set_error("engine: bad head configuration");
        return L2Q_ERR_ARG;
    }
    const int hs = c.dim / c.n_heads;
    const int kv_dim = hs * c.n_kv_heads;
    if (!gemv_shape_ok(wbits, group, 1, c.dim) || !gemv_shape_ok(wbits, group, 1, c.hidden_dim) ||
        !attention_shape_ok(c.n_heads, c.n_kv_heads, hs) || hs % 2 || c.dim > kNormThreads * kNormMaxPer ||
        !attention_exact_ok(max_steps <= 0 || max_steps > c.seq_len ? c.seq_len : max_steps)) {
        set_error("engine: unsupported shape (dim %d hidden %d heads %d group %d bits %d)", c.dim, c.hidden_dim,
                  c.n_heads, group, wbits);
        return L2Q_ERR_ARG;
    }
    l2q_engine* e = new (std::nothrow) l2q_engine();
    if (!e) { set_error("engine: out of host memory"); return L2Q_ERR_NOMEM; }
    e->cfg = c;
    e->wbits = wbits;
    e->G = group;
    e->hs = hs;
    e->kv_dim = kv_dim;
    e->max_t = (max_steps <= 0 || max_steps > c.seq_len) ? c.seq_len : max_steps;
    e->S = score_splits(e->max_t);
    hipError_t he = hipGetDevice(&e->device);
    if (he == hipSuccess) he = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
    int rc = he == hipSuccess ? build(e, weights, weights_bytes) : hip_fail(he, "engine: device/stream");
    if (rc) {
        release(e);
        delete e;
        return rc;
    }
    *out = e;
    return L2Q_OK;
}

int l2q_engine_forward(l2q_engine* e, int token, int pos, float* logits) {
    int rc = check_step(e, token, pos);
    if (rc) return rc;
    if ((rc = launch_step(e, token, pos, e->exec, 0))) return rc;
    if (logits)
        HIPCHK(hipMemcpyAsync(logits, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, e->stream),
               "copy logits");
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return L2Q_OK;
}

int l2q_engine_forward_argmax(l2q_engine* e, int token, int pos, int* next) {
    int rc = check_step(e, token, pos);
    if (rc) return rc;
    if (!next) { set_error("engine: null output"); return L2Q_ERR_ARG; }
    if ((rc = launch_step(e, token, pos, e->exec_am, 0))) return rc;
    HIPCHK(hipMemcpyAsync(e->h_am, e->am, sizeof(int), hipMemcpyDeviceToHost, e->stream), "copy argmax");
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    *next = *e->h_am;
    return L2Q_OK;
}

int l2q_engine_forward_debug(l2q_engine* e, int token, int pos, float* x_layers, float* logits) {
    int rc = check_step(e, token, pos);
    if (rc) return rc;
    if (!x_layers) { set_error("engine: null output"); return L2Q_ERR_ARG; }
    e->h_meta[0] = token;
    e->h_meta[1] = pos;
    HIPCHK(hipMemcpyAsync(e->meta, e->h_meta, 2 * sizeof(int), hipMemcpyHostToDevice, e->stream), "upload meta");
    std::vector<float> tmp(e->cfg.dim);
    if ((rc = enqueue_step(e, e->stream, x_layers, tmp.data(), false))) return rc;
    if (logits)
        HIPCHK(hipMemcpyAsync(logits, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, e->stream),
               "copy logits");
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return L2Q_OK;
}

int l2q_engine_time_steps(l2q_engine* e, const int* tokens, int pos0, int n_steps, double* elapsed_ms) {
    if (!e || !tokens || !elapsed_ms || n_steps <= 0) { set_error("engine: bad timing arguments"); return L2Q_ERR_ARG; }
    for (int i = 0; i < n_steps; i++) {
        int rc = check_step(e, tokens[i], pos0 + i);
        if (rc) return rc;
    }
    if (e->h_meta_slots < n_steps) {
        HIPCHK(hipHostFree(e->h_meta), "hipHostFree");
        e->h_meta = nullptr;
        HIPCHK(hipHostMalloc((void**)&e->h_meta, 2 * sizeof(int) * n_steps, hipHostMallocDefault), "hipHostMalloc");
        e->h_meta_slots = n_steps;
    }
    HIPCHK(hipEventRecord(e->ev0, e->stream), "hipEventRecord");
    for (int i = 0; i < n_steps; i++) {
        int rc = launch_step(e, tokens[i], pos0 + i, e->exec, i);
        if (rc) return rc;
    }
    HIPCHK(hipEventRecord(e->ev1, e->stream), "hipEventRecord");
    HIPCHK(hipEventSynchronize(e->ev1), "hipEventSynchronize");
    float ms = 0.0f;
    HIPCHK(hipEventElapsedTime(&ms, e->ev0, e->ev1), "hipEventElapsedTime");
    *elapsed_ms = ms;
    return L2Q_OK;
}

size_t l2q_engine_device_bytes(const l2q_engine* e) { return e ? e->wbytes + e->sbytes : 0; }

void l2q_engine_destroy(l2q_engine* e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    release(e);
    delete e;
}

}  // extern "C"
