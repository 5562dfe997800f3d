/* ref_runq_driver.c - compiles the reference CPU runner, unmodified, from
 * its own source file (v1-int8-vnni/runq.c under the reference checkout,
 * passed in as RUNQ_SOURCE by oracle/Makefile) and exposes its functions to
 * the test harness.  TEST INFRASTRUCTURE ONLY: used to pin the oracle and
 * as the reference CPU baseline; nothing in the product links it.
 *
 * The reference's main() is renamed so this file can add a C API; every
 * computation goes through the reference's own code.
 */
#define main runq_reference_main
#include RUNQ_SOURCE
#undef main

static Transformer g_t;
static int g_open = 0;

/* build_transformer (runq.c:280) on a QLL8 v1 file. */
int ref_open(char* checkpoint) {
    if (g_open) { free_transformer(&g_t); g_open = 0; }
    build_transformer(&g_t, checkpoint);
    g_open = 1;
    return g_t.config.vocab_size;
}

void ref_config(int out[7]) {
    const Config* c = &g_t.config;
    out[0] = c->dim; out[1] = c->hidden_dim; out[2] = c->n_layers; out[3] = c->n_heads;
    out[4] = c->n_kv_heads; out[5] = c->vocab_size; out[6] = c->seq_len;
}

/* forward (runq.c:320); returns the reference's logits buffer. */
float* ref_forward(int token, int pos) { return forward(&g_t, token, pos); }

/* Residual stream after the last forward (runq.c:325, RunState.x, which the
 * final rmsnorm overwrites in place: this is the normalised x). */
float* ref_state_x(void) { return g_t.state.x; }

void ref_close(void) {
    if (g_open) free_transformer(&g_t);
    g_open = 0;
}

/* quantize_act (runq.c:117), QBLOCK = 32. */
void ref_quantize_act(const float* x, int n, int8_t* xq, float* xs, float* xt) {
    quantize_act(x, n, xq, xs, xt);
}

/* matmul_q8 (runq.c:142) on caller buffers. */
void ref_matmul_q8(float* out, const int8_t* xq, const float* xs, const float* xt,
                   uint8_t* wq, float* ws, int rows, int cols) {
    QWeight w;
    w.q = wq; w.s = ws; w.rows = rows; w.cols = cols; w.nb = cols / QBLOCK;
    matmul_q8(out, xq, xs, xt, w);
}

/* rmsnorm (runq.c:294) and softmax (runq.c:307). */
void ref_rmsnorm(float* o, float* x, float* w, int n) { rmsnorm(o, x, w, n); }
void ref_softmax(float* x, int n) { softmax(x, n); }
int ref_sample_argmax(float* p, int n) { return sample_argmax(p, n); }
