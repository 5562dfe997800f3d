/* convert.c - llama2.c v0 fp32 checkpoint -> QLL8 / QLL4 checkpoint.
 *
 * The C form of the reference's offline tools tools/quantize_int8.py:64-126
 * and tools/quantize_int4.py:54-118: same input walk over the fp32 file
 * (v0-fp32/run.c:111-162: 28-byte Config header, tensors in order, the two
 * RoPE tables skipped, wcls present only when vocab_size < 0), same output
 * layout (qformat.h) and the same per-group quantizers (qll_quantize_row_q8
 * / _q4).  Differences, all opt-in:
 *   -g 64      group sizes other than 32 are written as version 3 (the
 *              group follows the config), which the reference tools cannot
 *              produce;
 *   -d 7       the INT4 scale divisor (the reference tool uses 8);
 *   -u         a shared-classifier checkpoint (vocab_size > 0) gets its
 *              embedding quantized as wcls and a negative vocab_size, so
 *              that runners which require an unshared classifier (runq.c:
 *              246-250) can load it.  Without -u the file mirrors the tool:
 *              vocab_size keeps its sign and wcls is omitted.
 *
 * usage: llama2q_convert in_fp32.bin out.bin [-b 8|4] [-g group] [-d div] [-u]
 */
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "qformat.h"

static void usage(void) {
    fprintf(stderr,
            "usage: llama2q_convert in_fp32.bin out.bin [options]\n"
            "  -b <int>   weight bits, 8 (QLL8) or 4 (QLL4); default 8\n"
            "  -g <int>   quantization group; default 32 (the reference tools' block)\n"
            "  -d <float> INT4 scale divisor (amax/d); default 8 as tools/quantize_int4.py\n"
            "  -u         write a shared classifier as an explicit (unshared) wcls\n");
    exit(EXIT_FAILURE);
}

typedef struct {
    FILE* out;
    int wbits, group;
    float div;
    uint8_t* qbuf;
} Writer;

static void put_bytes(Writer* w, const void* p, size_t n, const char* what) {
    if (n && fwrite(p, 1, n, w->out) != n) {
        fprintf(stderr, "write failed (%s): %s\n", what, strerror(errno));
        exit(EXIT_FAILURE);
    }
}

/* A quantized matrix: all weight bytes, then all scales (qformat.h). */
static void put_q(Writer* w, const float* m, size_t rows, size_t cols, const char* what) {
    const size_t rowb = qll_matrix_bytes(1, cols, w->wbits), nb = cols / (size_t)w->group;
    const size_t chunk = 256;   /* rows per pass: bounded buffers for any model size */
    float* scales = (float*)malloc(rows * nb * sizeof(float));
    if (!scales) { fprintf(stderr, "out of memory (%s)\n", what); exit(EXIT_FAILURE); }
    for (size_t r0 = 0; r0 < rows; r0 += chunk) {
        const size_t nr = rows - r0 < chunk ? rows - r0 : chunk;
        for (size_t r = 0; r < nr; r++) {
            const float* src = m + (r0 + r) * cols;
            uint8_t* q = w->qbuf + r * rowb;
            float* s = scales + (r0 + r) * nb;
            if (w->wbits == 8) qll_quantize_row_q8(src, (int)cols, w->group, q, s);
            else qll_quantize_row_q4(src, (int)cols, w->group, w->div, q, s);
        }
        put_bytes(w, w->qbuf, nr * rowb, what);
    }
    put_bytes(w, scales, rows * nb * sizeof(float), what);
    free(scales);
}

int main(int argc, char** argv) {
    if (argc < 3) usage();
    const char* in_path = argv[1];
    const char* out_path = argv[2];
    int wbits = 8, group = 32, unshare = 0;
    float div = 8.0f;
    for (int i = 3; i < argc; i++) {
        if (!strcmp(argv[i], "-u")) { unshare = 1; continue; }
        if (i + 1 >= argc || argv[i][0] != '-' || strlen(argv[i]) != 2) usage();
        switch (argv[i][1]) {
            case 'b': wbits = atoi(argv[++i]); break;
            case 'g': group = atoi(argv[++i]); break;
            case 'd': div = (float)atof(argv[++i]); break;
            default: usage();
        }
    }
    if ((wbits != 8 && wbits != 4) || group <= 0 || group % 2 || !(div > 0.0f)) usage();

    int fd = open(in_path, O_RDONLY);
    if (fd < 0) { fprintf(stderr, "cannot open %s: %s\n", in_path, strerror(errno)); return EXIT_FAILURE; }
    struct stat st;
    if (fstat(fd, &st) || st.st_size < 28) { fprintf(stderr, "%s: not a llama2.c checkpoint\n", in_path); return EXIT_FAILURE; }
    const size_t fsize = (size_t)st.st_size;
    const uint8_t* data = (const uint8_t*)mmap(NULL, fsize, PROT_READ, MAP_PRIVATE, fd, 0);
    if (data == MAP_FAILED) { fprintf(stderr, "mmap failed: %s\n", strerror(errno)); return EXIT_FAILURE; }

    int32_t cfg[7];
    memcpy(cfg, data, sizeof cfg);
    const int shared = cfg[5] > 0;
    l2q_config c = {cfg[0], cfg[1], cfg[2], cfg[3], cfg[4], abs(cfg[5]), cfg[6]};
    if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
        c.vocab_size <= 0 || c.seq_len <= 0 || c.dim % c.n_heads || c.n_heads % c.n_kv_heads ||
        c.dim % group || c.hidden_dim % group) {
        fprintf(stderr, "%s: config (dim %d hidden %d heads %d/%d) does not fit group %d\n", in_path, c.dim,
                c.hidden_dim, c.n_heads, c.n_kv_heads, group);
        return EXIT_FAILURE;
    }
    const size_t d = (size_t)c.dim, h = (size_t)c.hidden_dim, L = (size_t)c.n_layers, V = (size_t)c.vocab_size;
    const size_t hs = d / (size_t)c.n_heads, kv = d * (size_t)c.n_kv_heads / (size_t)c.n_heads;
    /* v0-fp32/run.c:111-142: element offsets of every tensor */
    const float* p = (const float*)(data + 28);
    const float *emb = p, *rms_att = emb + V * d, *wq = rms_att + L * d, *wk = wq + L * d * d;
    const float *wv = wk + L * kv * d, *wo = wv + L * kv * d, *rms_ffn = wo + L * d * d;
    const float *w1 = rms_ffn + L * d, *w2 = w1 + L * h * d, *w3 = w2 + L * d * h, *rms_final = w3 + L * h * d;
    const float* wcls = rms_final + d + (size_t)c.seq_len * hs;   /* two RoPE tables of seq_len*hs/2 */
    const size_t need = 28 + (size_t)((shared ? rms_final + d : wcls + V * d) - p) * sizeof(float);
    if (fsize < need) {
        fprintf(stderr, "%s: %zu bytes, the config needs %zu\n", in_path, fsize, need);
        return EXIT_FAILURE;
    }

    Writer w = {fopen(out_path, "wb"), wbits, group, div, NULL};
    if (!w.out) { fprintf(stderr, "cannot create %s: %s\n", out_path, strerror(errno)); return EXIT_FAILURE; }
    const size_t maxcols = d > h ? d : h;
    w.qbuf = (uint8_t*)malloc(256 * qll_matrix_bytes(1, maxcols, wbits));
    if (!w.qbuf) { fprintf(stderr, "out of memory\n"); return EXIT_FAILURE; }

    /* header: the tools' (magic, version, config with vocab sign kept), or
     * version 3 + group for other group sizes */
    const uint32_t magic = wbits == 8 ? QLL8_MAGIC : QLL4_MAGIC;
    const uint32_t version = group != 32 ? QLL_VERSION_GROUP : (wbits == 8 ? QLL_VERSION_Q8 : QLL_VERSION_Q4);
    int32_t ocfg[7];
    memcpy(ocfg, cfg, sizeof ocfg);
    if (shared && unshare) ocfg[5] = -ocfg[5];
    put_bytes(&w, &magic, 4, "header");
    put_bytes(&w, &version, 4, "header");
    put_bytes(&w, ocfg, sizeof ocfg, "header");
    if (version == QLL_VERSION_GROUP) {
        const uint32_t g = (uint32_t)group;
        put_bytes(&w, &g, 4, "header");
    }
    put_bytes(&w, emb, V * d * 4, "emb");
    put_bytes(&w, rms_att, L * d * 4, "rms_att");
    put_q(&w, wq, L * d, d, "wq");
    put_q(&w, wk, L * kv, d, "wk");
    put_q(&w, wv, L * kv, d, "wv");
    put_q(&w, wo, L * d, d, "wo");
    put_bytes(&w, rms_ffn, L * d * 4, "rms_ffn");
    put_q(&w, w1, L * h, d, "w1");
    put_q(&w, w2, L * d, h, "w2");
    put_q(&w, w3, L * h, d, "w3");
    put_bytes(&w, rms_final, d * 4, "rms_final");
    if (!shared) put_q(&w, wcls, V, d, "wcls");
    else if (unshare) put_q(&w, emb, V, d, "wcls");
    if (fclose(w.out)) { fprintf(stderr, "close failed: %s\n", strerror(errno)); return EXIT_FAILURE; }
    free(w.qbuf);
    munmap((void*)data, fsize);
    close(fd);
    fprintf(stderr, "wrote %s (%s, group %d%s)\n", out_path, wbits == 8 ? "QLL8" : "QLL4", group,
            shared ? (unshare ? ", classifier unshared" : ", shared classifier omitted") : "");
    return EXIT_SUCCESS;
}
