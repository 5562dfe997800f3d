// engine.hip - the decode engine behind l2q_engine_* (include/l2q.h).
//
// Device layout (one weight arena, one state arena, both hipMalloc'd once):
//   emb        fp32 [V][d]            rms_att / rms_ffn fp32 [L][d], rms_final [d]
//   qkv_w      [L][d + 2kv][d*bits/8] rows of wq, wk, wv of a layer, back to back
//   qkv_s      [L][d + 2kv][d/G]      fp32 scales in the same row order
//   wo_w/s     [L][d][...]            as in the file
//   w13_w/s    [L][2h][...]           rows of w1 and w3 interleaved (w1[i], w3[i], ...)
//   w2_w/s     [L][d][...]
//   wcls_w/s   [V][...]
//   INT8 weights are stored signed (the file's +128 bias removed at load).
//   vcache     fp32 [L][n_kv_heads][max_t][hs]
//   kcache     fp32 [L][n_kv_heads][hs/4][max_t][4]: float4 columns of consecutive
//              positions contiguous (k_index), so the attention, one position per
//              lane, reads K with coalesced loads
// Concatenating wq|wk|wv and interleaving w1/w3 turns 5 GEMV launches per
// layer into 2 with 12288- and 22016-row grids at the 7B shape, and lets the
// SwiGLU run in the GEMV's epilogue.
//
// A layer is five launches (runq.c:335-415):
//   QKV   residual add + RMSNorm + quantize prologue, RoPE + KV append epilogue
//   attention scores, softmax, p*V in the exact order: one kernel up to
//         attention_fused_max() positions, two (scores; softmax + p*V) beyond
//   wo    quantize prologue
//   W13   residual add + RMSNorm + quantize prologue, SwiGLU epilogue
//   W2    quantize prologue
// The residual stream ping-pongs between xa and xb: a norm prologue reads one
// and its workgroup 0 persists x + resid into the other.
//
// One decode step (runq.c:320-421) is captured once into a hipGraph; the
// token and position are read from device memory (`meta`), so every step
// replays the same graph after an 8-byte upload (as v5-cuda-fused/run.cu:
// 671-695 does).
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "launch.h"
#include "qformat.h"

struct l2q_engine {
    l2q_config cfg;
    int wbits, G, max_t, kv_dim, hs, S;
    int flags;               // L2Q_ENGINE_* options
    int device;
    hipStream_t stream = nullptr;
    // captured steps [argmax][long context]: the long-context graphs exist
    // only when the cache outgrows g_switch positions (fp32 cache: the
    // two-kernel attention beyond attention_fused_max(); int8 cache: the
    // split-context attention beyond L2Q_KV8_SPLIT_FROM)
    int g_switch = 0;
    hipGraph_t graph[2][2] = {};
    hipGraphExec_t exec[2][2] = {};
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
    float *xa, *xb, *q, *att, *wo_out, *hb, *ffn_out, *logits;
    float *kcache, *vcache, *rope, *scores;
    int8_t *k8, *v8;         // L2Q_ENGINE_KV_INT8: [L][n_kv][max_t][hs]
    float *ks, *vs;          //   scales [L][n_kv][max_t]
    float* kvf;              //   the position's rotated k and v rows [2][kv_dim]
    int *meta, *am;
    float *tout, *tx, *tkv;  // l2q_engine_time_gemv outputs (2h, d, 2kv floats): the state stays untouched
    // the one-kernel step (step.h): used when L2Q_ENGINE_STEP_KERNEL is set and the shape has it
    bool step = false;
    l2q::StepArgs sa{};
    int step_grid = 0;
    size_t step_lds_bytes = 0;
    unsigned* sync = nullptr;   // grp | top | rel | err | epoch (StepSync)
    size_t sync_bytes = 0;
    float* dbg = nullptr;       // [L+1][d]: the residual stream of forward_debug
    // the split-context attentions (L2Q_ENGINE_ATTN_SPLIT, the int8 KV
    // cache): partials [n_heads][aS][hs + 2] and per-head counters (left
    // zeroed)
    float* apart = nullptr;
    unsigned* acnt = nullptr;
    int aS = 0;
    int* h_meta = nullptr;   // pinned {token, pos} slots
    int h_meta_slots = 0;
    int* h_am = nullptr;     // pinned argmax result, then the step kernel's error word
    // batched prefill (allocated at the first l2q_engine_prefill): T tokens per chunk
    char* pfarena = nullptr;
    int pf_T = 0;
    float *pf_xa, *pf_xb, *pf_qkv, *pf_att, *pf_wo, *pf_ffn, *pf_scores;
    int8_t *pf_xqp, *pf_xqh;           // GEMM operands: d-wide, and w2's h-wide one (written by w1|w3)
    float* pf_kvst;                    // int8 KV cache: the chunk's rotated k, v rows [2][n_kv][pf_T][hs]
    float* pf_apart;                   //   and its split attention's partials, per query of a chunk
    unsigned* pf_acnt;                 //   and merge counters (zeroed; the kernel leaves them zeroed)
    l2q::PfRecord *pf_rec, *pf_rech;
    int* pf_tok;
};

using namespace l2q;

namespace {

// Positions from which the tolerance mode runs the split-context attention:
// measured on MI355X at the 7B shape, the exact one-kernel attention takes
// 8.8 us at 256 positions and grows ~0.017 us per position, the split form
// stays near 9 us (they cross near 280).
constexpr int kAttnSplitFrom = L2Q_ATTN_SPLIT_FROM;


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

// The GEMVs of the step: arguments, prologue and epilogue of matrix `kind`
// of layer l (kClassifier: the final norm + classifier, l ignored).
enum GemvKind { kQkv = 0, kWo = 1, kW13 = 2, kW2 = 3, kClassifier = 4 };

struct StepGemv {
    GemvArgs a{};
    int pro = kQuant, epi = kStore;
};

StepGemv step_gemv(const l2q_engine* e, int kind, int l) {
    const l2q_config& c = e->cfg;
    const int d = c.dim, h = c.hidden_dim, kv = e->kv_dim, G = e->G;
    const int qkv_rows = d + 2 * kv;
    const size_t nbd = (size_t)d / G, nbh = (size_t)h / G;
    StepGemv g;
    GemvArgs& a = g.a;
    switch (kind) {
        case kQkv: {   // x = (l == 0 ? emb[token] : xa + ffn_out) -> xb; RMSNorm; q, k, v; RoPE + append
            a.out = e->q;
            a.w = e->qkv_w + (size_t)l * qkv_rows * e->rowb_d;
            a.ws = e->qkv_s + (size_t)l * qkv_rows * nbd;
            a.rows = qkv_rows;
            a.cols = d;
            a.x_in = e->xa;
            a.emb = l == 0 ? e->emb : nullptr;
            a.resid = l == 0 ? nullptr : e->ffn_out;
            a.x_out = e->xb;
            a.norm_w = e->rms_att + (size_t)l * d;
            a.meta = e->meta;
            a.dim = d; a.kv_dim = kv; a.hs = e->hs; a.max_t = e->max_t;
            a.kcache = e->kcache + (size_t)l * kv * e->max_t;
            a.vcache = e->vcache + (size_t)l * kv * e->max_t;
            a.rope = e->rope;
            a.k_il = 1;
            if (e->flags & L2Q_ENGINE_KV_INT8) {   // k, v rows to the staging row, quantized by the attention
                a.kcache = e->kvf; a.vcache = e->kvf + kv; a.max_t = 1; a.kv_stage = 1; a.k_il = 0;
            }
            g.pro = kNorm; g.epi = kRopeKV;
            break;
        }
        case kWo:   // quantize the attention output in the prologue
            a.out = e->wo_out;
            a.w = e->wo_w + (size_t)l * d * e->rowb_d;
            a.ws = e->wo_s + (size_t)l * d * nbd;
            a.rows = d;
            a.cols = d;
            a.x_in = e->att;
            break;
        case kW13:   // x = xb + wo_out -> xa; RMSNorm; SwiGLU(w1 x, w3 x) -> hb
            a.out = e->hb;
            a.w = e->w13_w + (size_t)l * 2 * h * e->rowb_d;
            a.ws = e->w13_s + (size_t)l * 2 * h * nbd;
            a.rows = 2 * h;
            a.cols = d;
            a.x_in = e->xb;
            a.resid = e->wo_out;
            a.x_out = e->xa;
            a.norm_w = e->rms_ffn + (size_t)l * d;
            a.meta = e->meta;
            g.pro = kNorm; g.epi = kSwiglu;
            break;
        case kW2:   // quantize hb in the prologue
            a.out = e->ffn_out;
            a.w = e->w2_w + (size_t)l * d * e->rowb_h;
            a.ws = e->w2_s + (size_t)l * d * nbh;
            a.rows = d;
            a.cols = h;
            a.x_in = e->hb;
            break;
        default:   // final RMSNorm of xa + ffn_out, classifier
            a.out = e->logits;
            a.w = e->wcls_w;
            a.ws = e->wcls_s;
            a.rows = c.vocab_size;
            a.cols = d;
            a.x_in = e->xa;
            a.resid = e->ffn_out;
            a.norm_w = e->rms_final;
            a.meta = e->meta;
            g.pro = kNorm;
            break;
    }
    return g;
}

int launch_step_gemv(const l2q_engine* e, int kind, int l, hipStream_t st) {
    const StepGemv g = step_gemv(e, kind, l);
    return launch_gemv_fused(e->wbits, e->G, g.pro, g.epi, g.a, st);
}

// Enqueue one decode step on `st` (captured or eager).  If `dbg_x` is set
// (eager diagnostic mode) the residual stream after the embedding and after
// each layer is copied to it.
int enqueue_step(l2q_engine* e, hipStream_t st, float* dbg_x, float* dbg_tmp, bool argmax, bool fused) {
    const l2q_config& c = e->cfg;
    const int d = c.dim, kv = e->kv_dim;
    int rc;
    for (int l = 0; l < c.n_layers; l++) {
        float* kc = e->kcache + (size_t)l * kv * e->max_t;
        float* vc = e->vcache + (size_t)l * kv * e->max_t;
        if ((rc = launch_step_gemv(e, kQkv, l, st))) return rc;
        if (dbg_x && l == 0) HIPCHK(hipMemcpyAsync(dbg_x, e->xb, d * sizeof(float), hipMemcpyDeviceToHost, st), "copy x");
        if (e->flags & L2Q_ENGINE_KV_INT8) {
            const size_t co = (size_t)l * kv * e->max_t, so = (size_t)l * c.n_kv_heads * e->max_t;
            // append the staged k, v rows and attend in one kernel: one
            // workgroup per head up to L2Q_KV8_SPLIT_FROM positions, split
            // over the context beyond
            if (fused)
                rc = launch_attention_kv8(e->q, e->k8 + co, e->v8 + co, e->ks + so, e->vs + so, e->att, e->scores,
                                          e->meta, 0, c.n_heads, c.n_kv_heads, e->hs, e->max_t, st, e->kvf,
                                          e->kvf + kv);
            else
                rc = launch_attention_kv8_split(e->q, e->kvf, e->kvf + kv, e->k8 + co, e->v8 + co, e->ks + so,
                                                e->vs + so, e->att, e->apart, e->acnt, e->aS, e->meta, 0, c.n_heads,
                                                c.n_kv_heads, e->hs, e->max_t, st);
        } else if ((e->flags & L2Q_ENGINE_ATTN_SPLIT) && !fused) {
            rc = launch_attention_flash(e->q, kc, vc, e->att, e->apart, e->acnt, e->aS, e->meta, 0, c.n_heads,
                                        c.n_kv_heads, e->hs, e->max_t, 1, st);
        } else {
            rc = launch_attention_exact(e->q, kc, vc, e->att, e->scores, e->S, e->meta, 0, c.n_heads,
                                        c.n_kv_heads, e->hs, e->max_t, st, 1, 0, fused ? 1 : 0, 1);
        }
        if (rc) return rc;
        if ((rc = launch_step_gemv(e, kWo, l, st))) return rc;
        if ((rc = launch_step_gemv(e, kW13, l, st))) return rc;
        if ((rc = launch_step_gemv(e, kW2, l, st))) return rc;
        if (dbg_x) {
            float* dst = dbg_x + (size_t)(l + 1) * d;
            HIPCHK(hipMemcpyAsync(dst, e->xa, d * sizeof(float), hipMemcpyDeviceToHost, st), "copy x");
            HIPCHK(hipMemcpyAsync(dbg_tmp, e->ffn_out, d * sizeof(float), hipMemcpyDeviceToHost, st), "copy ffn");
            HIPCHK(hipStreamSynchronize(st), "sync");
            for (int i = 0; i < d; i++) dst[i] = dst[i] + dbg_tmp[i];   // the add the next norm performs
        }
    }
    if ((rc = launch_step_gemv(e, kClassifier, 0, st))) return rc;
    if (argmax) return launch_argmax(e->logits, c.vocab_size, e->am, st);
    return L2Q_OK;
}

// Whether the one-kernel step serves this engine (L2Q_ENGINE_STEP_KERNEL): INT4 weights in groups of
// 64, dim-wide rows of 2 sweeps, w2 rows of 5-6 sweeps, heads of 128 with
// the fp32 cache, a cache the fused attention holds, staged outputs within
// kStepStage per wave, LDS within the CU's and one resident workgroup per CU.
int step_setup(l2q_engine* e, int ncu) {
    const l2q_config& c = e->cfg;
    e->step = false;
    if (!(e->flags & L2Q_ENGINE_STEP_KERNEL) || (e->flags & (L2Q_ENGINE_KV_INT8 | L2Q_ENGINE_ATTN_SPLIT)) || ncu <= 0 ||
        ncu % 8)
        return L2Q_OK;
    if (e->wbits != 4 || e->G != 64 || !step_shape_ok(c.dim, c.hidden_dim, e->hs)) return L2Q_OK;
    if (e->max_t > attention_fused_max()) return L2Q_OK;
    // row pairs per workgroup within the fold areas; staged outputs per wave
    const int rows_max = std::max(std::max(c.dim + 2 * e->kv_dim, 2 * c.hidden_dim), c.vocab_size);
    const int pairs_wg = ((rows_max + 1) / 2 + ncu - 1) / ncu;
    if (pairs_wg > kStepPairsCap || (c.dim / 2 + ncu - 1) / ncu > kStepPairsCapH) return L2Q_OK;
    if (2 * ((pairs_wg + kStepCompute - 1) / kStepCompute) > kStepStage) return L2Q_OK;
    const int items = c.n_heads * (e->hs / kStepAttnSlice);
    if (kStepAttnSlice * ((items + ncu - 1) / ncu) > kStepStage) return L2Q_OK;
    const size_t lds = step_lds_bytes();
    int maxlds = 0;
    if (hipDeviceGetAttribute(&maxlds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, e->device) != hipSuccess ||
        lds > (size_t)maxlds)
        return L2Q_OK;
    int per_cu = 0;
    int rc = step_prepare(lds, &per_cu);
    if (rc) return rc;
    if (per_cu < 1) return L2Q_OK;
    StepArgs& a = e->sa;
    a.qkv_w = e->qkv_w; a.wo_w = e->wo_w; a.w13_w = e->w13_w; a.w2_w = e->w2_w; a.wcls_w = e->wcls_w;
    a.qkv_s = e->qkv_s; a.wo_s = e->wo_s; a.w13_s = e->w13_s; a.w2_s = e->w2_s; a.wcls_s = e->wcls_s;
    a.emb = e->emb; a.rms_att = e->rms_att; a.rms_ffn = e->rms_ffn; a.rms_final = e->rms_final; a.rope = e->rope;
    a.xa = e->xa; a.xb = e->xb; a.q = e->q; a.att = e->att; a.wo_out = e->wo_out; a.hb = e->hb;
    a.ffn_out = e->ffn_out; a.logits = e->logits; a.kcache = e->kcache; a.vcache = e->vcache;
    a.meta = e->meta;
    a.dbg_x = nullptr;
    a.sync.grp = e->sync;
    a.sync.top = e->sync + 8 * 16;
    a.sync.rel = e->sync + 9 * 16;
    a.sync.err = a.sync.rel + (size_t)ncu * 16;
    a.sync.epoch = a.sync.err + 16;
    a.d = c.dim; a.h = c.hidden_dim; a.L = c.n_layers; a.V = c.vocab_size;
    a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.hs = e->hs; a.kv = e->kv_dim; a.max_t = e->max_t;
    a.rowb_d = (int)e->rowb_d; a.rowb_h = (int)e->rowb_h;
    a.nbar = step_phases(c.n_layers) - 1;
    e->step_grid = ncu;
    e->step_lds_bytes = lds;
    e->step = true;
    return L2Q_OK;
}

int launch_step_kernel(l2q_engine* e, hipStream_t st, float* dbg) {
    StepArgs a = e->sa;
    a.dbg_x = dbg;
    return launch_step_kernel(a, e->step_grid, e->step_lds_bytes, st);
}

// A timed-out step leaves the barrier state inconsistent: report it and
// reset the state (zeroed counters, epoch 0) for the next launch.
int step_check(l2q_engine* e) {
    if (!e->step || e->h_am[1] == 0) return L2Q_OK;
    (void)hipMemsetAsync(e->sync, 0, e->sync_bytes, e->stream);
    (void)hipStreamSynchronize(e->stream);
    set_error("engine: a grid barrier of the decode step timed out (not every workgroup was resident)");
    return L2Q_ERR_HIP;
}

int copy_step_err(l2q_engine* e) {
    if (!e->step) return L2Q_OK;
    HIPCHK(hipMemcpyAsync(e->h_am + 1, e->sa.sync.err, sizeof(int), hipMemcpyDeviceToHost, e->stream), "copy step error");
    return L2Q_OK;
}

int capture(l2q_engine* e, bool argmax, bool fused, hipGraph_t* g, hipGraphExec_t* ex) {
    HIPCHK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    int rc;
    if (e->step) {
        rc = launch_step_kernel(e, e->stream, nullptr);
        if (!rc && argmax) rc = launch_argmax(e->logits, e->cfg.vocab_size, e->am, e->stream);
    } else {
        rc = enqueue_step(e, e->stream, nullptr, nullptr, argmax, fused);
    }
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
    for (int a = 0; a < 2; a++)
        for (int l = 0; l < 2; l++) {
            if (e->exec[a][l]) (void)hipGraphExecDestroy(e->exec[a][l]);
            if (e->graph[a][l]) (void)hipGraphDestroy(e->graph[a][l]);
        }
    if (e->ev0) (void)hipEventDestroy(e->ev0);
    if (e->ev1) (void)hipEventDestroy(e->ev1);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    if (e->warena) (void)hipFree(e->warena);
    if (e->sarena) (void)hipFree(e->sarena);
    if (e->pfarena) (void)hipFree(e->pfarena);
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
    std::vector<uint8_t> stage_w(2 * h * e->rowb_d);
    std::vector<float> stage_s(2 * h * nbd);
    for (size_t l = 0; l < L; l++) {
        uint8_t* qw = e->qkv_w + l * qkv_rows * e->rowb_d;
        float* qs = e->qkv_s + l * qkv_rows * nbd;
        if ((rc = copy_h2d(qw, F + lay.wq + l * d * e->rowb_d, d * e->rowb_d))) return rc;
        if ((rc = copy_h2d(qw + d * e->rowb_d, F + lay.wk + l * kv * e->rowb_d, kv * e->rowb_d))) return rc;
        if ((rc = copy_h2d(qw + (d + kv) * e->rowb_d, F + lay.wv + l * kv * e->rowb_d, kv * e->rowb_d))) return rc;
        if ((rc = copy_h2d(qs, F + lay.wq_s + l * d * nbd * 4, d * nbd * 4))) return rc;
        if ((rc = copy_h2d(qs + d * nbd, F + lay.wk_s + l * kv * nbd * 4, kv * nbd * 4))) return rc;
        if ((rc = copy_h2d(qs + (d + kv) * nbd, F + lay.wv_s + l * kv * nbd * 4, kv * nbd * 4))) return rc;
        // w1/w3 rows interleaved: row 2i = w1[i], row 2i+1 = w3[i]
        for (size_t i = 0; i < h; i++) {
            std::memcpy(stage_w.data() + (2 * i) * e->rowb_d, F + lay.w1 + (l * h + i) * e->rowb_d, e->rowb_d);
            std::memcpy(stage_w.data() + (2 * i + 1) * e->rowb_d, F + lay.w3 + (l * h + i) * e->rowb_d, e->rowb_d);
            std::memcpy(stage_s.data() + (2 * i) * nbd, F + lay.w1_s + (l * h + i) * nbd * 4, nbd * 4);
            std::memcpy(stage_s.data() + (2 * i + 1) * nbd, F + lay.w3_s + (l * h + i) * nbd * 4, nbd * 4);
        }
        if ((rc = copy_h2d(e->w13_w + l * 2 * h * e->rowb_d, stage_w.data(), stage_w.size()))) return rc;
        if ((rc = copy_h2d(e->w13_s + l * 2 * h * nbd, stage_s.data(), stage_s.size() * 4))) return rc;
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
    const size_t o_xa = sa.take(d * 4), o_xb = sa.take(d * 4), o_q = sa.take(d * 4), o_att = sa.take(d * 4);
    const size_t o_wo = sa.take(d * 4), o_hb = sa.take(h * 4), o_ffn = sa.take(d * 4);
    const size_t o_logits = sa.take(V * 4);
    const bool kv8 = e->flags & L2Q_ENGINE_KV_INT8;
    const size_t kvfloats = kv8 ? 0 : L * kv * (size_t)e->max_t;
    const size_t o_kc = sa.take(kvfloats * 4), o_vc = sa.take(kvfloats * 4);
    const size_t kv8n = kv8 ? L * kv * (size_t)e->max_t : 0, kv8s = kv8 ? L * (size_t)c.n_kv_heads * e->max_t : 0;
    const size_t o_k8 = sa.take(kv8n), o_v8 = sa.take(kv8n), o_ks = sa.take(kv8s * 4), o_vs = sa.take(kv8s * 4);
    const size_t o_kvf = sa.take(kv8 ? 2 * kv * 4 : 0);
    const size_t o_rope = sa.take((size_t)e->max_t * e->hs * 4);
    const size_t o_sc = sa.take((size_t)c.n_heads * e->max_t * 4);
    const size_t o_meta = sa.take(2 * sizeof(int)), o_am = sa.take(sizeof(int));
    const size_t o_tout = sa.take((size_t)2 * h * 4 + V * 4), o_tx = sa.take(d * 4), o_tkv = sa.take(2 * kv * 4);
    int ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, e->device) != hipSuccess || ncu < 8) ncu = 0;
    e->sync_bytes = (size_t)(8 * 16 + 16 + (size_t)(ncu > 0 ? ncu : 8) * 16 + 16 + 16) * sizeof(unsigned);
    const size_t o_sync = sa.take(e->sync_bytes), o_dbg = sa.take((L + 1) * d * 4);
    const bool asplit = e->flags & L2Q_ENGINE_ATTN_SPLIT;
    e->aS = asplit || kv8 ? attention_flash_splits(c.n_heads, e->max_t, ncu) : 0;
    const size_t o_apart = sa.take(e->aS ? attention_flash_part_floats(c.n_heads, e->aS, e->hs) * 4 : 0);
    const size_t o_acnt = sa.take(e->aS ? (size_t)c.n_heads * sizeof(unsigned) : 0);
    e->sbytes = align_up(sa.used, 256);
    HIPCHK(hipMalloc(&e->sarena, e->sbytes), "hipMalloc(state)");
    char* S_ = e->sarena;
    e->xa = (float*)(S_ + o_xa); e->xb = (float*)(S_ + o_xb); e->q = (float*)(S_ + o_q); e->att = (float*)(S_ + o_att);
    e->wo_out = (float*)(S_ + o_wo); e->hb = (float*)(S_ + o_hb); e->ffn_out = (float*)(S_ + o_ffn);
    e->logits = (float*)(S_ + o_logits);
    e->kcache = (float*)(S_ + o_kc); e->vcache = (float*)(S_ + o_vc); e->rope = (float*)(S_ + o_rope);
    e->scores = (float*)(S_ + o_sc);
    e->k8 = (int8_t*)(S_ + o_k8); e->v8 = (int8_t*)(S_ + o_v8);
    e->ks = (float*)(S_ + o_ks); e->vs = (float*)(S_ + o_vs); e->kvf = (float*)(S_ + o_kvf);
    e->meta = (int*)(S_ + o_meta); e->am = (int*)(S_ + o_am);
    e->tout = (float*)(S_ + o_tout); e->tx = (float*)(S_ + o_tx); e->tkv = (float*)(S_ + o_tkv);
    e->sync = (unsigned*)(S_ + o_sync); e->dbg = (float*)(S_ + o_dbg);
    e->apart = (float*)(S_ + o_apart); e->acnt = (unsigned*)(S_ + o_acnt);
    // zero-fill the state (outside any graph) so unused cache rows are defined
    HIPCHK(hipMemsetAsync(e->sarena, 0, e->sbytes, e->stream), "hipMemset(state)");

    std::vector<float> rope((size_t)e->max_t * e->hs);
    l2q_rope_table(rope.data(), e->max_t, e->hs);
    HIPCHK(hipMemcpyAsync(e->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice, e->stream), "copy rope");
    HIPCHK(hipStreamSynchronize(e->stream), "sync(build)");

    e->h_meta_slots = 1;
    HIPCHK(hipHostMalloc((void**)&e->h_meta, 2 * sizeof(int) * e->h_meta_slots, hipHostMallocDefault), "hipHostMalloc");
    HIPCHK(hipHostMalloc((void**)&e->h_am, 2 * sizeof(int), hipHostMallocDefault), "hipHostMalloc");
    if ((rc = step_setup(e, ncu))) return rc;
    HIPCHK(hipEventCreate(&e->ev0), "hipEventCreate");
    HIPCHK(hipEventCreate(&e->ev1), "hipEventCreate");
    // short contexts: one-kernel attention where the head size has it; the
    // tolerance mode (L2Q_ENGINE_ATTN_SPLIT) switches to the split-context
    // kernel from kAttnSplitFrom positions, where it overtakes the exact
    // one (below, the exact kernel is the faster and the more exact)
    e->g_switch = kv8 ? L2Q_KV8_SPLIT_FROM
                      : asplit ? std::min(attention_fused_max(), kAttnSplitFrom) : attention_fused_max();
    const bool fused = e->step || kv8 || attention_fused_ok(e->hs);
    const bool need_long = !e->step && (!fused || e->max_t > e->g_switch);
    for (int a = 0; a < 2; a++) {
        if (fused && (rc = capture(e, a, true, &e->graph[a][0], &e->exec[a][0]))) return rc;
        if (need_long && (rc = capture(e, a, false, &e->graph[a][1], &e->exec[a][1]))) return rc;
    }
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

// The captured step for this position: the short-context graph up to
// g_switch positions, the long-context one beyond.
hipGraphExec_t step_graph(const l2q_engine* e, bool argmax, int pos) {
    hipGraphExec_t const* g = e->exec[argmax ? 1 : 0];
    return g[0] && (!g[1] || pos + 1 <= e->g_switch) ? g[0] : g[1];
}

int launch_step(l2q_engine* e, int token, int pos, hipGraphExec_t ex, int slot) {
    int* hm = e->h_meta + 2 * slot;
    hm[0] = token;
    hm[1] = pos;
    HIPCHK(hipMemcpyAsync(e->meta, hm, 2 * sizeof(int), hipMemcpyHostToDevice, e->stream), "upload meta");
    HIPCHK(hipGraphLaunch(ex, e->stream), "hipGraphLaunch");
    return L2Q_OK;
}

// Prefill buffers for chunks of up to pf_T tokens.
int prefill_alloc(l2q_engine* e) {
    if (e->pfarena) return L2Q_OK;
    const l2q_config& c = e->cfg;
    const size_t T = (size_t)(e->max_t < kPfMaxTokens ? e->max_t : kPfMaxTokens);
    const size_t d = c.dim, h = c.hidden_dim, kv = e->kv_dim, qkv = d + 2 * kv;
    const size_t kmax = d > h ? d : h, nbmax = kmax / e->G;
    Arena a;
    const size_t o_xa = a.take(T * d * 4), o_xb = a.take(T * d * 4), o_qkv = a.take(T * qkv * 4);
    const size_t o_att = a.take(T * d * 4), o_wo = a.take(T * d * 4);
    const size_t o_ffn = a.take(T * d * 4), o_sc = a.take(T * c.n_heads * (size_t)attn_b_pitch(e->max_t) * 4);
    const size_t o_xqp = a.take(T * kmax), o_rec = a.take(T * nbmax * sizeof(PfRecord));
    const size_t o_xqh = a.take(T * h), o_rech = a.take(T * (h / e->G) * sizeof(PfRecord));
    const size_t o_tok = a.take(T * 4);
    const bool kv8 = e->flags & L2Q_ENGINE_KV_INT8;
    const size_t o_kvst = a.take(kv8 ? 2 * T * kv * 4 : 0);
    const size_t o_apart = a.take(kv8 && e->aS ? T * attention_flash_part_floats(c.n_heads, e->aS, e->hs) * 4 : 0);
    const size_t o_acnt = a.take(kv8 && e->aS ? T * c.n_heads * sizeof(unsigned) : 0);
    HIPCHK(hipMalloc(&e->pfarena, align_up(a.used, 256)), "hipMalloc(prefill)");
    char* P = e->pfarena;
    e->pf_xa = (float*)(P + o_xa); e->pf_xb = (float*)(P + o_xb); e->pf_qkv = (float*)(P + o_qkv);
    e->pf_att = (float*)(P + o_att); e->pf_wo = (float*)(P + o_wo);
    e->pf_ffn = (float*)(P + o_ffn); e->pf_scores = (float*)(P + o_sc);
    e->pf_xqp = (int8_t*)(P + o_xqp); e->pf_rec = (PfRecord*)(P + o_rec);
    e->pf_xqh = (int8_t*)(P + o_xqh); e->pf_rech = (PfRecord*)(P + o_rech);
    e->pf_tok = (int*)(P + o_tok);
    e->pf_kvst = kv8 ? (float*)(P + o_kvst) : nullptr;
    e->pf_apart = kv8 && e->aS ? (float*)(P + o_apart) : nullptr;
    e->pf_acnt = kv8 && e->aS ? (unsigned*)(P + o_acnt) : nullptr;
    if (e->pf_acnt) HIPCHK(hipMemset(e->pf_acnt, 0, T * c.n_heads * sizeof(unsigned)), "hipMemset(prefill counters)");
    e->pf_T = (int)T;
    return L2Q_OK;
}

// T tokens at positions pos0.. through every layer at once: the same
// operations as T decode steps (so the KV rows and the last position's
// logits are bit-identical), with the weights streamed once per chunk.
int prefill_chunk(l2q_engine* e, const int* tokens, int T, int pos0, bool want_logits) {
    const l2q_config& c = e->cfg;
    const int d = c.dim, h = c.hidden_dim, kv = e->kv_dim, G = e->G, bits = e->wbits;
    const int qkv_rows = d + 2 * kv;
    const size_t nbd = (size_t)d / G, nbh = (size_t)h / G;
    hipStream_t st = e->stream;
    int rc;
    HIPCHK(hipMemcpyAsync(e->pf_tok, tokens, T * sizeof(int), hipMemcpyHostToDevice, st), "upload tokens");
    if ((rc = launch_pf_embed(e->emb, e->pf_tok, e->pf_xa, d, T, st))) return rc;
    // every quantizing producer writes the GEMM operand (permuted q, records) itself
    const PfOperand pod{e->pf_xqp, e->pf_rec, bits, d, T}, poh{e->pf_xqh, e->pf_rech, bits, h, T};
    auto gemm = [&](const uint8_t* w, const float* ws, int rows, const PfOperand& in, float* out,
                    const PfRope* rp = nullptr, const PfOperand* sw = nullptr) {
        return launch_pf_gemm(bits, G, w, ws, rows, in.K, in.xqp, in.rec, T, out, rows, st, rp, sw);
    };
    const bool kv8 = e->flags & L2Q_ENGINE_KV_INT8;
    // int8 KV cache: queries whose decode step runs the one-workgroup-per-
    // head kernel (positions up to the engine's switch), the rest split
    int nfused = 0;
    if (kv8)
        while (nfused < T && step_graph(e, false, pos0 + nfused) == e->exec[0][0]) nfused++;
    for (int l = 0; l < c.n_layers; l++) {
        // x = (l == 0 ? emb rows : xa + ffn) -> xb; RMSNorm; q, k, v; RoPE + append; attention
        if ((rc = launch_rmsnorm_quant(e->pf_xa, nullptr, nullptr, l == 0 ? nullptr : e->pf_ffn, e->pf_xb,
                                       e->rms_att + (size_t)l * d, d, G, nullptr, nullptr, st, T, &pod)))
            return rc;
        const uint8_t* wqkv = e->qkv_w + (size_t)l * qkv_rows * e->rowb_d;
        const float* sqkv = e->qkv_s + (size_t)l * qkv_rows * nbd;
        if (kv8) {
            // q, and the rotated k, v rows to the chunk's staging; the decode
            // step's int8 append (k_kv8_append) of every row; then each query's
            // attention as its decode step runs it (the appended rows read back)
            const size_t co = (size_t)l * kv * e->max_t, so = (size_t)l * c.n_kv_heads * e->max_t;
            float* stk = e->pf_kvst;
            float* stv = e->pf_kvst + (size_t)e->pf_T * kv;
            const PfRope rp{e->rope, stk, stv, pos0, d, kv, e->hs, e->pf_T, 0, 0};
            if ((rc = gemm(wqkv, sqkv, qkv_rows, pod, e->pf_qkv, &rp))) return rc;
            if ((rc = launch_kv8_append(stk, stv, e->k8 + co, e->v8 + co, e->ks + so, e->vs + so, nullptr, nullptr,
                                        pos0, c.n_kv_heads, e->hs, e->max_t, st, T, e->pf_T)))
                return rc;
            if (nfused &&
                (rc = launch_attention_kv8(e->pf_qkv, e->k8 + co, e->v8 + co, e->ks + so, e->vs + so, e->pf_att,
                                           nullptr, nullptr, pos0, c.n_heads, c.n_kv_heads, e->hs, e->max_t, st,
                                           nullptr, nullptr, nfused, qkv_rows, d)))
                return rc;
            if (nfused < T &&
                (rc = launch_attention_kv8_split(e->pf_qkv + (size_t)nfused * qkv_rows, nullptr, nullptr, e->k8 + co,
                                                 e->v8 + co, e->ks + so, e->vs + so, e->pf_att + (size_t)nfused * d,
                                                 e->pf_apart, e->pf_acnt, e->aS, nullptr, pos0 + nfused, c.n_heads,
                                                 c.n_kv_heads, e->hs, e->max_t, st, T - nfused, qkv_rows, d)))
                return rc;
            if ((rc = launch_quantize(e->pf_att, T * d, G, nullptr, nullptr, st, &pod))) return rc;
        } else {
            float* kc = e->kcache + (size_t)l * kv * e->max_t;
            float* vc = e->vcache + (size_t)l * kv * e->max_t;
            // q, k, v rows with RoPE and the KV append fused into the GEMM's stores
            const PfRope rp{e->rope, kc, vc, pos0, d, kv, e->hs, e->max_t, 1, pos0};
            if ((rc = gemm(wqkv, sqkv, qkv_rows, pod, e->pf_qkv, &rp))) return rc;
            // attention, its output quantized into the wo operand
            if ((rc = launch_attention_prefill(e->pf_qkv, kc, vc, e->pf_att, e->pf_scores, pos0, c.n_heads,
                                               c.n_kv_heads, e->hs, e->max_t, st, T, qkv_rows, 1, G, &pod)))
                return rc;
        }
        // wo
        if ((rc = gemm(e->wo_w + (size_t)l * d * e->rowb_d, e->wo_s + (size_t)l * d * nbd, d, pod, e->pf_wo))) return rc;
        // x = xb + wo -> xa; RMSNorm; SwiGLU(w1 x, w3 x); w2
        if ((rc = launch_rmsnorm_quant(e->pf_xb, nullptr, nullptr, e->pf_wo, e->pf_xa, e->rms_ffn + (size_t)l * d, d,
                                       G, nullptr, nullptr, st, T, &pod)))
            return rc;
        // w1|w3 with SwiGLU + Q8 in its stores: w2's operand, no h13 in HBM
        if ((rc = gemm(e->w13_w + (size_t)l * 2 * h * e->rowb_d, e->w13_s + (size_t)l * 2 * h * nbd, 2 * h, pod,
                       nullptr, nullptr, &poh)))
            return rc;
        if ((rc = gemm(e->w2_w + (size_t)l * d * e->rowb_h, e->w2_s + (size_t)l * d * nbh, d, poh, e->pf_ffn))) return rc;
    }
    if (!want_logits) return L2Q_OK;
    // the last position: final RMSNorm of xa + ffn, classifier
    GemvArgs ca{};
    ca.out = e->logits;
    ca.w = e->wcls_w;
    ca.ws = e->wcls_s;
    ca.rows = c.vocab_size;
    ca.cols = d;
    ca.x_in = e->pf_xa + (size_t)(T - 1) * d;
    ca.resid = e->pf_ffn + (size_t)(T - 1) * d;
    ca.norm_w = e->rms_final;
    ca.meta = e->meta;
    return launch_gemv_fused(bits, G, kNorm, kStore, ca, st);
}

}  // namespace

extern "C" {

int l2q_engine_prefill(l2q_engine* e, const int* tokens, int n, int pos0, float* logits) {
    if (!e || !tokens || n < 1) { set_error("engine: bad prefill arguments"); return L2Q_ERR_ARG; }
    if (pos0 < 0 || pos0 + n > e->max_t) {
        set_error("engine: prefill positions %d..%d outside the KV cache (max_steps %d)", pos0, pos0 + n - 1,
                  e->max_t);
        return L2Q_ERR_STATE;
    }
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= e->cfg.vocab_size) { set_error("engine: token %d out of range", tokens[i]); return L2Q_ERR_ARG; }
    int rc;
    if ((rc = prefill_alloc(e))) return rc;
    for (int i0 = 0; i0 < n; i0 += e->pf_T) {
        const int T = n - i0 < e->pf_T ? n - i0 : e->pf_T;
        if ((rc = prefill_chunk(e, tokens + i0, T, pos0 + i0, i0 + T == n))) return rc;
    }
    if (logits)
        HIPCHK(hipMemcpyAsync(logits, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, e->stream),
               "copy logits");
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return L2Q_OK;
}


int l2q_engine_create(const l2q_config* cfg, const void* weights, size_t weights_bytes, int wbits, int group,
                      int max_steps, l2q_engine** out) {
    return l2q_engine_create_ex(cfg, weights, weights_bytes, wbits, group, max_steps, 0, out);
}

int l2q_engine_create_ex(const l2q_config* cfg, const void* weights, size_t weights_bytes, int wbits, int group,
                         int max_steps, int flags, l2q_engine** out) {
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
        !attention_shape_ok(c.n_heads, c.n_kv_heads, hs) || hs % 2 || c.dim > kNormThreads * kNormMaxPer) {
        set_error("engine: unsupported shape (dim %d hidden %d heads %d group %d bits %d)", c.dim, c.hidden_dim,
                  c.n_heads, group, wbits);
        return L2Q_ERR_ARG;
    }
    if (!attention_exact_ok(max_steps <= 0 || max_steps > c.seq_len ? c.seq_len : max_steps)) {
        set_error("engine: too many cached positions (max_steps %d, seq_len %d; the exact attention holds at most %d)",
                  max_steps, c.seq_len, attention_exact_max());
        return L2Q_ERR_ARG;
    }
    const int steps = max_steps <= 0 || max_steps > c.seq_len ? c.seq_len : max_steps;
    if ((flags & ~(L2Q_ENGINE_KV_INT8 | L2Q_ENGINE_STEP_KERNEL | L2Q_ENGINE_ATTN_SPLIT)) ||
        ((flags & L2Q_ENGINE_KV_INT8) && !kv8_shape_ok(c.n_heads, c.n_kv_heads, hs, steps)) ||
        ((flags & L2Q_ENGINE_ATTN_SPLIT) && ((flags & L2Q_ENGINE_KV_INT8) || !attention_flash_ok(hs)))) {
        set_error("engine: unsupported flags %d for this shape (int8 KV needs head_size %% 16 == 0, <= 8192 steps; "
                  "the split-context attention needs the fp32 cache and head_size 48, 64 or 128)",
                  flags);
        return L2Q_ERR_ARG;
    }
    l2q_engine* e = new (std::nothrow) l2q_engine();
    if (!e) { set_error("engine: out of host memory"); return L2Q_ERR_NOMEM; }
    e->flags = flags;
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
    if ((rc = launch_step(e, token, pos, step_graph(e, false, pos), 0))) return rc;
    if (logits)
        HIPCHK(hipMemcpyAsync(logits, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, e->stream),
               "copy logits");
    if ((rc = copy_step_err(e))) return rc;
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return step_check(e);
}

int l2q_engine_forward_argmax(l2q_engine* e, int token, int pos, int* next) {
    int rc = check_step(e, token, pos);
    if (rc) return rc;
    if (!next) { set_error("engine: null output"); return L2Q_ERR_ARG; }
    if ((rc = launch_step(e, token, pos, step_graph(e, true, pos), 0))) return rc;
    HIPCHK(hipMemcpyAsync(e->h_am, e->am, sizeof(int), hipMemcpyDeviceToHost, e->stream), "copy argmax");
    if ((rc = copy_step_err(e))) return rc;
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    if ((rc = step_check(e))) return rc;
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
    if (e->step) {
        if ((rc = launch_step_kernel(e, e->stream, e->dbg))) return rc;
        HIPCHK(hipMemcpyAsync(x_layers, e->dbg, (size_t)(e->cfg.n_layers + 1) * e->cfg.dim * sizeof(float),
                              hipMemcpyDeviceToHost, e->stream),
               "copy x");
        if ((rc = copy_step_err(e))) return rc;
    } else {
        std::vector<float> tmp(e->cfg.dim);
        if ((rc = enqueue_step(e, e->stream, x_layers, tmp.data(), false, step_graph(e, false, pos) == e->exec[0][0])))
            return rc;
    }
    if (logits)
        HIPCHK(hipMemcpyAsync(logits, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, e->stream),
               "copy logits");
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    return step_check(e);
}

// Pinned (token, pos) slots for n steps enqueued before any completes.
int ensure_meta_slots(l2q_engine* e, int n_steps) {
    if (e->h_meta_slots < n_steps) {
        HIPCHK(hipHostFree(e->h_meta), "hipHostFree");
        e->h_meta = nullptr;
        HIPCHK(hipHostMalloc((void**)&e->h_meta, 2 * sizeof(int) * n_steps, hipHostMallocDefault), "hipHostMalloc");
        e->h_meta_slots = n_steps;
    }
    return L2Q_OK;
}

int l2q_engine_time_steps(l2q_engine* e, const int* tokens, int pos0, int n_steps, double* elapsed_ms) {
    if (!e || !tokens || !elapsed_ms || n_steps <= 0) { set_error("engine: bad timing arguments"); return L2Q_ERR_ARG; }
    for (int i = 0; i < n_steps; i++) {
        int rc = check_step(e, tokens[i], pos0 + i);
        if (rc) return rc;
    }
    int rc = ensure_meta_slots(e, n_steps);
    if (rc) return rc;
    HIPCHK(hipEventRecord(e->ev0, e->stream), "hipEventRecord");
    for (int i = 0; i < n_steps; i++) {
        if ((rc = launch_step(e, tokens[i], pos0 + i, step_graph(e, false, pos0 + i), i))) return rc;
    }
    HIPCHK(hipEventRecord(e->ev1, e->stream), "hipEventRecord");
    rc = copy_step_err(e);
    if (rc) return rc;
    HIPCHK(hipEventSynchronize(e->ev1), "hipEventSynchronize");
    HIPCHK(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
    float ms = 0.0f;
    HIPCHK(hipEventElapsedTime(&ms, e->ev0, e->ev1), "hipEventElapsedTime");
    *elapsed_ms = ms;
    return step_check(e);
}

int l2q_engine_time_gemv(l2q_engine* e, int kind, int n_launches, double* elapsed_ms) {
    if (!e || !elapsed_ms || n_launches <= 0 || kind < L2Q_GEMV_QKV || kind > L2Q_GEMV_CLASSIFIER) {
        set_error("engine: bad GEMV timing arguments");
        return L2Q_ERR_ARG;
    }
    const int L = e->cfg.n_layers;
    auto launch = [&](int i) {
        StepGemv g = step_gemv(e, kind, i % L);
        // outputs to the timing area: the decode state is left as it was
        g.a.out = e->tout;
        if (g.a.x_out) g.a.x_out = e->tx;
        if (g.epi == kRopeKV) {
            g.a.kcache = e->tkv; g.a.vcache = e->tkv + e->kv_dim; g.a.max_t = 1; g.a.kv_stage = 1; g.a.k_il = 0;
        }
        return launch_gemv_fused(e->wbits, e->G, g.pro, g.epi, g.a, e->stream);
    };
    int rc;
    for (int i = 0; i < L; i++)   // warm: every layer's launch once
        if ((rc = launch(i))) return rc;
    HIPCHK(hipEventRecord(e->ev0, e->stream), "hipEventRecord");
    for (int i = 0; i < n_launches; i++)
        if ((rc = launch(i))) return rc;
    HIPCHK(hipEventRecord(e->ev1, e->stream), "hipEventRecord");
    HIPCHK(hipEventSynchronize(e->ev1), "hipEventSynchronize");
    float ms = 0.0f;
    HIPCHK(hipEventElapsedTime(&ms, e->ev0, e->ev1), "hipEventElapsedTime");
    *elapsed_ms = ms;
    return L2Q_OK;
}

int l2q_engine_attention_splits(const l2q_engine* e) { return e ? e->aS : 0; }

int l2q_engine_uses_step_kernel(const l2q_engine* e) { return e && e->step ? 1 : 0; }

size_t l2q_engine_device_bytes(const l2q_engine* e) { return e ? e->wbytes + e->sbytes : 0; }

void l2q_engine_destroy(l2q_engine* e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    release(e);
    delete e;
}

}  // extern "C"
