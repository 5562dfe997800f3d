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
    if (g_open == 1) free_transformer(&g_t);
    else if (g_open == 2) free_run_state(&g_t.state);
    g_open = 0;
    build_transformer(&g_t, checkpoint);
    g_open = 1;
    return g_t.config.vocab_size;
}

/* The same set-up from a QLL8 v1 image already in memory (no file):
 * header checks as read_checkpoint (runq.c:259-268), then the reference's
 * memory_map_weights and malloc_run_state.  `data` must outlive the model. */
int ref_open_memory(uint8_t* data, size_t size) {
    if (g_open == 1) free_transformer(&g_t);
    else if (g_open == 2) free_run_state(&g_t.state);
    g_open = 0;
    uint32_t magic, version;
    if (size < 36) return -1;
    memcpy(&magic, data, 4);
    memcpy(&version, data + 4, 4);
    if (magic != QMAGIC || version != QVERSION) return -1;
    memcpy(&g_t.config, data + 8, sizeof(Config));
    int shared = g_t.config.vocab_size > 0 ? 1 : 0;
    g_t.config.vocab_size = abs(g_t.config.vocab_size);
    g_t.fd = -1;
    g_t.data = MAP_FAILED;
    g_t.file_size = (ssize_t)size;
    memory_map_weights(&g_t.weights, &g_t.config, data + 2 * sizeof(uint32_t) + sizeof(Config), shared);
    malloc_run_state(&g_t.state, &g_t.config);
    g_open = 2;
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
    if (g_open == 1) free_transformer(&g_t);
    else if (g_open == 2) free_run_state(&g_t.state);
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

/* ---- the reference's tokenizer and sampler (runq.c:426-667) ---------- */

static Tokenizer g_tok;
static int g_tok_open = 0;

void ref_tok_open(char* path, int vocab_size) {
    if (g_tok_open) free_tokenizer(&g_tok);
    build_tokenizer(&g_tok, path, vocab_size);
    g_tok_open = 1;
}

/* encode (runq.c:500); returns the number of tokens */
int ref_tok_encode(char* text, int bos, int eos, int* tokens) {
    int n = 0;
    encode(&g_tok, text, (int8_t)bos, (int8_t)eos, tokens, &n);
    return n;
}

char* ref_tok_decode(int prev, int token) { return decode(&g_tok, prev, token); }

void ref_tok_close(void) {
    if (g_tok_open) free_tokenizer(&g_tok);
    g_tok_open = 0;
}

static Sampler g_smp;
static int g_smp_open = 0;

void ref_sampler_open(int vocab_size, float temperature, float topp, unsigned long long seed) {
    if (g_smp_open) free_sampler(&g_smp);
    build_sampler(&g_smp, vocab_size, temperature, topp, seed);
    g_smp_open = 1;
}

/* sample (runq.c:652); modifies logits like the reference */
int ref_sample(float* logits) { return sample(&g_smp, logits); }

unsigned long long ref_sampler_state(void) { return g_smp.rng_state; }

void ref_sampler_close(void) {
    if (g_smp_open) free_sampler(&g_smp);
    g_smp_open = 0;
}
