/* run.c - drop-in command-line runner for QLL8 / QLL4 checkpoints.
 *
 * Same usage, flags, defaults and output as the reference runners
 * (runq.c:799-870, v5-cuda-fused/run.cu:1063-1171):
 *
 *   llama2q_run <checkpoint> [-t temp] [-p topp] [-s seed] [-n steps]
 *               [-i prompt] [-z tokenizer] [-m generate|chat] [-y system]
 *
 * The checkpoint is mmapped and handed to the GPU engine through the C ABI
 * (l2q.h); every position is one l2q_engine_forward call, exactly where the
 * reference calls forward() (runq.c:698, 781).  Greedy decoding (-t 0) uses
 * the device-side argmax so only the chosen id crosses PCIe.
 */
#define _GNU_SOURCE
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "l2q.h"
#include "qformat.h"
#include "sampler.h"
#include "tokenizer.h"

static void die(const char* what, const char* detail) {
    fprintf(stderr, "%s%s%s\n", what, detail ? ": " : "", detail ? detail : "");
    exit(EXIT_FAILURE);
}

static long time_in_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_REALTIME, &ts);
    return ts.tv_sec * 1000 + ts.tv_nsec / 1000000;
}

typedef struct {
    l2q_engine* engine;
    l2q_sampler* sampler;
    float* logits;
} decoder;

/* forward + sample for one position; logits are fetched only when needed. */
static int step(decoder* d, int token, int pos, int want_next) {
    int next = -1;
    if (!want_next) {
        if (l2q_engine_forward(d->engine, token, pos, NULL) != L2Q_OK) die("forward failed", l2q_last_error());
        return -1;
    }
    if (d->sampler->temperature == 0.0f) {
        if (l2q_engine_forward_argmax(d->engine, token, pos, &next) != L2Q_OK) die("forward failed", l2q_last_error());
        return next;
    }
    if (l2q_engine_forward(d->engine, token, pos, d->logits) != L2Q_OK) die("forward failed", l2q_last_error());
    return sampler_sample(d->sampler, d->logits);
}

/* Generation loop of runq.c:681-718: prompt forcing, stop at BOS.
 *
 * "achieved tok/s" keeps runq's formula, (pos - 1) / elapsed (runq.c:
 * 710-716).  runq starts its clock when step 1 ends; when the forced prompt
 * positions run as one batched prefill there is no separate step 1, so the
 * clock starts before that prefill (the rate then also carries step 1's
 * work: it can only read lower than runq's).  A second line gives the rate
 * of the positions decoded after the prefill alone. */
static void generate(decoder* d, l2q_tokenizer* tk, const char* prompt, int steps) {
    if (prompt == NULL) prompt = "";
    int* toks = (int*)malloc((strlen(prompt) + 3) * sizeof(int));
    int n = tok_encode(tk, prompt, 1, 0, toks);
    if (n < 1) die("something is wrong, expected at least 1 prompt token", NULL);
    long start = 0, decode_start = 0;
    int token = toks[0], pos = 0, next, decode_pos0 = 0, done = 0;
    /* the forced prompt positions in one batched pass (the same KV cache and
     * text as forcing them one by one, runq.c:695-700), then the loop */
    const int npf = n - 1 < steps ? n - 1 : steps;
    if (npf > 1) {
        start = time_in_ms();
        if (l2q_engine_prefill(d->engine, toks, npf, 0, NULL) != L2Q_OK) die("prefill failed", l2q_last_error());
        for (; pos < npf; pos++) {
            next = toks[pos + 1];
            if (next == 1) { done = 1; pos++; break; }
            tok_print_piece(tok_decode(tk, token, next));
            token = next;
        }
        fflush(stdout);
        decode_start = time_in_ms();
        decode_pos0 = pos;
    }
    while (!done && pos < steps) {
        int forced = pos < n - 1;
        next = step(d, token, pos, !forced);
        if (forced) next = toks[pos + 1];
        pos++;
        if (next == 1) break;
        tok_print_piece(tok_decode(tk, token, next));
        fflush(stdout);
        token = next;
        if (start == 0) { start = time_in_ms(); decode_start = start; decode_pos0 = 1; }
    }
    printf("\n");
    long end = time_in_ms();
    if (pos > 1 && start != 0)
        fprintf(stderr, "achieved tok/s: %f\n", (pos - 1) / (double)(end - start) * 1000);
    if (npf > 1 && pos > decode_pos0 && end > decode_start)
        fprintf(stderr, "decode tok/s (after the %d-position prefill): %f\n", npf,
                (pos - decode_pos0) / (double)(end - decode_start) * 1000);
    free(toks);
}

/* read_stdin of runq.c:720-729: at end of input the buffer keeps what it
 * held, so a chat whose input has run out repeats the last user turn. */
static void read_line(const char* guide, char* buf, size_t n) {
    printf("%s", guide);
    fflush(stdout);
    if (fgets(buf, (int)n, stdin) != NULL) {
        size_t len = strlen(buf);
        if (len && buf[len - 1] == '\n') buf[len - 1] = 0;
    }
}

/* Llama-2 chat loop of runq.c:731-794 (the same templates, turn switching
 * on id 2 and printing; it runs for `steps` positions). */
static void chat(decoder* d, l2q_tokenizer* tk, const char* cli_user, const char* cli_system,
                 int steps) {
    char system_prompt[512] = {0}, user_prompt[512] = {0}, rendered[1152];
    int* toks = (int*)malloc(1152 * sizeof(int));
    int n = 0, user_idx = 0, user_turn = 1, next = 0, token = 0, pos = 0;
    while (pos < steps) {
        if (user_turn) {
            if (pos == 0) {
                if (cli_system == NULL) read_line("Enter system prompt (optional): ", system_prompt, sizeof system_prompt);
                else snprintf(system_prompt, sizeof system_prompt, "%s", cli_system);
            }
            if (pos == 0 && cli_user != NULL) snprintf(user_prompt, sizeof user_prompt, "%s", cli_user);
            else read_line("User: ", user_prompt, sizeof user_prompt);
            if (pos == 0 && system_prompt[0] != 0)
                snprintf(rendered, sizeof rendered, "[INST] <<SYS>>\n%s\n<</SYS>>\n\n%s [/INST]",
                         system_prompt, user_prompt);
            else
                snprintf(rendered, sizeof rendered, "[INST] %s [/INST]", user_prompt);
            n = tok_encode(tk, rendered, 1, 0, toks);
            user_idx = 0;
            user_turn = 0;
            printf("Assistant: ");
        }
        token = user_idx < n ? toks[user_idx++] : next;
        if (token == 2) user_turn = 1;
        next = step(d, token, pos, 1);
        pos++;
        if (user_idx >= n && next != 2) {
            tok_print_piece(tok_decode(tk, token, next));
            fflush(stdout);
        }
        if (next == 2) printf("\n");
    }
    printf("\n");
    free(toks);
}

static void usage(void) {
    fprintf(stderr, "Usage:   llama2q_run <checkpoint> [options]\n");
    fprintf(stderr, "Example: llama2q_run llama2-7b-q4.bin -n 256 -i \"Once upon a time\"\n");
    fprintf(stderr, "Options:\n");
    fprintf(stderr, "  -t <float>  temperature in [0,inf], default 1.0\n");
    fprintf(stderr, "  -p <float>  p value in top-p (nucleus) sampling in [0,1] default 0.9\n");
    fprintf(stderr, "  -s <int>    random seed, default time(NULL)\n");
    fprintf(stderr, "  -n <int>    number of steps to run for, default 256. 0 = max_seq_len\n");
    fprintf(stderr, "  -i <string> input prompt\n");
    fprintf(stderr, "  -z <string> optional path to custom tokenizer\n");
    fprintf(stderr, "  -m <string> mode: generate|chat, default: generate\n");
    fprintf(stderr, "  -y <string> (optional) system prompt in chat mode\n");
    fprintf(stderr, "  -k <int>    KV cache element bits: 32 (default) or 8 (the reference's INT8_KV build)\n");
    exit(EXIT_FAILURE);
}

int main(int argc, char** argv) {
    const char* ckpt = NULL;
    const char* tok_path = "tokenizer.bin";
    float temperature = 1.0f, topp = 0.9f;
    int steps = 256;
    const char* prompt = NULL;
    unsigned long long seed = 0;
    const char* mode = "generate";
    const char* system_prompt = NULL;
    int kv_bits = 32;

    if (argc >= 2) ckpt = argv[1]; else usage();
    for (int i = 2; i < argc; i += 2) {
        if (i + 1 >= argc || argv[i][0] != '-' || strlen(argv[i]) != 2) usage();
        switch (argv[i][1]) {
            case 't': temperature = (float)atof(argv[i + 1]); break;
            case 'p': topp = (float)atof(argv[i + 1]); break;
            case 's': seed = (unsigned long long)atoi(argv[i + 1]); break;
            case 'n': steps = atoi(argv[i + 1]); break;
            case 'i': prompt = argv[i + 1]; break;
            case 'z': tok_path = argv[i + 1]; break;
            case 'm': mode = argv[i + 1]; break;
            case 'y': system_prompt = argv[i + 1]; break;
            case 'k': kv_bits = atoi(argv[i + 1]); break;
            default: usage();
        }
    }
    if (seed <= 0) seed = (unsigned int)time(NULL);
    if (temperature < 0.0f) temperature = 0.0f;
    if (topp < 0.0f || 1.0f < topp) topp = 0.9f;
    if (steps < 0) steps = 0;
    if (kv_bits != 32 && kv_bits != 8) usage();

    char err[256];
    qll_file f;
    if (qll_open(ckpt, &f, err, sizeof err) != 0) die(err, NULL);
    if (f.h.shared_weights) die("shared weights not supported", NULL);
    if (steps == 0 || steps > f.h.cfg.seq_len) steps = f.h.cfg.seq_len;

    l2q_engine* engine = NULL;
    if (l2q_engine_create_ex(&f.h.cfg, f.weights, f.weights_bytes, f.h.wbits, f.h.group, steps,
                             kv_bits == 8 ? L2Q_ENGINE_KV_INT8 : 0, &engine) != L2Q_OK)
        die("engine init failed", l2q_last_error());
    qll_close(&f);   /* the engine holds device copies of every tensor */

    l2q_tokenizer tk;
    if (tok_load(&tk, tok_path, f.h.cfg.vocab_size, err, sizeof err) != 0) die(err, NULL);
    l2q_sampler sampler;
    if (sampler_init(&sampler, f.h.cfg.vocab_size, temperature, topp, seed) != 0) die("malloc failed!", NULL);
    decoder d = {engine, &sampler, (float*)malloc((size_t)f.h.cfg.vocab_size * sizeof(float))};

    if (strcmp(mode, "generate") == 0) generate(&d, &tk, prompt, steps);
    else if (strcmp(mode, "chat") == 0) chat(&d, &tk, prompt, system_prompt, steps);
    else { fprintf(stderr, "unknown mode: %s\n", mode); usage(); }

    free(d.logits);
    sampler_free(&sampler);
    tok_free(&tk);
    l2q_engine_destroy(engine);
    return 0;
}
