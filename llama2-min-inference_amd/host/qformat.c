/* qformat.c - QLL8/QLL4 layout, header I/O, mmap reader, offline quantizers
 * and the deterministic random-init checkpoint writer. */
#define _GNU_SOURCE
#include "qformat.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static void set_err(char* err, size_t n, const char* fmt, const char* a, long b) {
    if (err && n) snprintf(err, n, fmt, a, b);
}

size_t qll_matrix_bytes(size_t rows, size_t cols, int wbits) {
    return wbits == 4 ? rows * cols / 2 : rows * cols;
}

/* Layout of tensors, in the order of runq.c:235-252 (memory_map_weights). */
int qll_layout_compute(const l2q_config* c, int wbits, int group, qll_layout* o) {
    if (c->dim <= 0 || c->hidden_dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 ||
        c->n_kv_heads <= 0 || c->vocab_size <= 0 || c->seq_len <= 0)
        return -1;
    if (wbits != 8 && wbits != 4) return -1;
    if (group <= 0 || (group % 16) != 0) return -1;
    if (c->dim % c->n_heads || c->n_heads % c->n_kv_heads) return -1;
    if (c->dim % group || c->hidden_dim % group) return -1;
    const size_t d = (size_t)c->dim, h = (size_t)c->hidden_dim, L = (size_t)c->n_layers;
    const size_t kv = d * (size_t)c->n_kv_heads / (size_t)c->n_heads;
    const size_t V = (size_t)c->vocab_size;
    size_t p = 0;
#define F32(name, n) do { o->name = p; p += (size_t)(n) * 4; } while (0)
#define QM(name, rows, cols) do { o->name = p; p += qll_matrix_bytes(rows, cols, wbits); \
        o->name##_s = p; p += (size_t)(rows) * ((cols) / (size_t)group) * 4; } while (0)
    F32(emb, V * d);
    F32(rms_att, L * d);
    QM(wq, L * d, d);
    QM(wk, L * kv, d);
    QM(wv, L * kv, d);
    QM(wo, L * d, d);
    F32(rms_ffn, L * d);
    QM(w1, L * h, d);
    QM(w2, L * d, h);
    QM(w3, L * h, d);
    F32(rms_final, d);
    QM(wcls, V, d);
#undef F32
#undef QM
    o->total = p;
    return 0;
}

size_t qll_write_header(void* dst, const l2q_config* c, int wbits, int group) {
    uint8_t* b = (uint8_t*)dst;
    uint32_t magic = wbits == 4 ? QLL4_MAGIC : QLL8_MAGIC;
    uint32_t version = group == 32 ? (wbits == 4 ? QLL_VERSION_Q4 : QLL_VERSION_Q8)
                                   : QLL_VERSION_GROUP;
    int32_t cfg[7] = {c->dim, c->hidden_dim, c->n_layers, c->n_heads, c->n_kv_heads,
                      -c->vocab_size /* unshared classifier */, c->seq_len};
    memcpy(b, &magic, 4);
    memcpy(b + 4, &version, 4);
    memcpy(b + 8, cfg, 28);
    if (version == QLL_VERSION_GROUP) {
        uint32_t g = (uint32_t)group;
        memcpy(b + 36, &g, 4);
        return 40;
    }
    return 36;
}

/* Header checks of runq.c:259-268 / v5-cuda-fused/run.cu:1126-1132. */
int qll_parse_header(const void* data, size_t n, qll_header* h, char* err, size_t errlen) {
    const uint8_t* b = (const uint8_t*)data;
    if (n < 36) { set_err(err, errlen, "%struncated header (%ld bytes)", "", (long)n); return L2Q_ERR_FORMAT; }
    uint32_t magic, version;
    int32_t cfg[7];
    memcpy(&magic, b, 4);
    memcpy(&version, b + 4, 4);
    memcpy(cfg, b + 8, 28);
    memset(h, 0, sizeof(*h));
    if (magic == QLL8_MAGIC) h->wbits = 8;
    else if (magic == QLL4_MAGIC) h->wbits = 4;
    else {
        if (err && errlen) snprintf(err, errlen, "bad magic/version (got %08x v%u)", magic, version);
        return L2Q_ERR_FORMAT;
    }
    if (version == QLL_VERSION_GROUP) {
        if (n < 40) { set_err(err, errlen, "%struncated header (%ld bytes)", "", (long)n); return L2Q_ERR_FORMAT; }
        uint32_t g;
        memcpy(&g, b + 36, 4);
        h->group = (int)g;
        h->header_bytes = 40;
    } else if ((h->wbits == 8 && version == QLL_VERSION_Q8) ||
               (h->wbits == 4 && version == QLL_VERSION_Q4)) {
        h->group = 32;
        h->header_bytes = 36;
    } else {
        if (err && errlen) snprintf(err, errlen, "bad magic/version (got %08x v%u)", magic, version);
        return L2Q_ERR_FORMAT;
    }
    h->cfg.dim = cfg[0];
    h->cfg.hidden_dim = cfg[1];
    h->cfg.n_layers = cfg[2];
    h->cfg.n_heads = cfg[3];
    h->cfg.n_kv_heads = cfg[4];
    h->shared_weights = cfg[5] > 0 ? 1 : 0;
    h->cfg.vocab_size = abs(cfg[5]);
    h->cfg.seq_len = cfg[6];
    return L2Q_OK;
}

int qll_open(const char* path, qll_file* f, char* err, size_t errlen) {
    memset(f, 0, sizeof(*f));
    f->fd = -1;
    int fd = open(path, O_RDONLY);
    if (fd < 0) { set_err(err, errlen, "Couldn't open file %s%.0ld", path, 0); return L2Q_ERR_ARG; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); set_err(err, errlen, "stat failed on %s%.0ld", path, 0); return L2Q_ERR_ARG; }
    size_t size = (size_t)st.st_size;
    uint8_t head[40] = {0};
    ssize_t got = pread(fd, head, sizeof(head), 0);
    if (got < 0) got = 0;
    int rc = qll_parse_header(head, (size_t)got, &f->h, err, errlen);
    if (rc) { close(fd); return rc; }
    void* m = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) { close(fd); set_err(err, errlen, "mmap failed%s (%ld)", "", (long)errno); return L2Q_ERR_ARG; }
    f->fd = fd;
    f->data = (const uint8_t*)m;
    f->file_size = size;
    f->weights = f->data + f->h.header_bytes;
    f->weights_bytes = size - f->h.header_bytes;
    return L2Q_OK;
}

void qll_close(qll_file* f) {
    if (f->data) munmap((void*)f->data, f->file_size);
    if (f->fd >= 0) close(f->fd);
    f->data = NULL;
    f->fd = -1;
}

/* ---------------- quantizers ------------------------------------------- */

void qll_quantize_row_q8(const float* w, int cols, int group, uint8_t* q, float* s) {
    for (int b = 0; b < cols / group; b++) {
        const float* wb = w + (size_t)b * group;
        float amax = 0.0f;
        for (int j = 0; j < group; j++) { float a = fabsf(wb[j]); if (a > amax) amax = a; }
        float sc = amax / 127.0f;
        if (sc == 0.0f) sc = 1e-8f;
        for (int j = 0; j < group; j++) {
            float r = rintf(wb[j] / sc);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[(size_t)b * group + j] = (uint8_t)((int)r + 128);
        }
        s[b] = sc;
    }
}

void qll_quantize_row_q4(const float* w, int cols, int group, float divisor,
                         uint8_t* q, float* s) {
    for (int b = 0; b < cols / group; b++) {
        const float* wb = w + (size_t)b * group;
        float amax = 0.0f;
        for (int j = 0; j < group; j++) { float a = fabsf(wb[j]); if (a > amax) amax = a; }
        float sc = amax / divisor;
        if (sc == 0.0f) sc = 1e-8f;
        for (int j = 0; j < group; j += 2) {
            float r0 = rintf(wb[j] / sc), r1 = rintf(wb[j + 1] / sc);
            r0 = r0 > 7.0f ? 7.0f : (r0 < -8.0f ? -8.0f : r0);
            r1 = r1 > 7.0f ? 7.0f : (r1 < -8.0f ? -8.0f : r1);
            uint8_t n0 = (uint8_t)((int)r0 & 0xF), n1 = (uint8_t)((int)r1 & 0xF);
            q[((size_t)b * group + j) / 2] = (uint8_t)(n0 | (n1 << 4));
        }
        s[b] = sc;
    }
}

/* ---------------- deterministic synthetic data ------------------------- */

static inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return splitmix64(splitmix64(seed) ^ (stream * 0xD1B54A32D192ED03ull));
}

static inline float gauss_from_key(uint64_t key, uint64_t index) {
    uint64_t h = splitmix64(key + (index >> 1));
    float u1 = (float)((h >> 40) + 1) * (1.0f / 16777216.0f);          /* (0, 1] */
    float u2 = (float)((h >> 8) & 0xFFFFFFu) * (1.0f / 16777216.0f);   /* [0, 1) */
    float r = sqrtf(-2.0f * logf(u1));
    float th = 6.28318530717958647692f * u2;
    return (index & 1) ? r * sinf(th) : r * cosf(th);
}

float qll_gauss(uint64_t seed, uint64_t stream, uint64_t index) {
    return gauss_from_key(stream_key(seed, stream), index);
}

void qll_gauss_fill(float* dst, size_t n, uint64_t seed, uint64_t stream,
                    uint64_t index0, float sigma) {
    uint64_t key = stream_key(seed, stream);
    for (size_t i = 0; i < n; i++) dst[i] = sigma * gauss_from_key(key, index0 + i);
}

int qll_uniform_int(uint64_t seed, uint64_t stream, uint64_t index, int lo, int hi) {
    uint64_t h = splitmix64(stream_key(seed, stream) + index);
    return lo + (int)((h >> 11) % (uint64_t)(hi - lo));
}

size_t qll_synth_size(const l2q_config* c, int wbits, int group) {
    qll_layout lay;
    if (qll_layout_compute(c, wbits, group, &lay)) return 0;
    return (group == 32 ? 36 : 40) + lay.total;
}

/* Stream ids of the tensors of a synthetic model. */
enum { S_EMB = 1, S_WQ = 3, S_WK, S_WV, S_WO, S_W1 = 8, S_W2, S_W3, S_WCLS = 12 };

/* Fill row r of a [rows][cols] matrix stream: elements come in Box-Muller
 * pairs (2k, 2k+1) sharing one (u1, u2) draw, so each pair costs one log,
 * one sqrt and one sincos; values equal qll_gauss(seed, stream, r*cols+j). */
static void gauss_row(float* row, size_t cols, uint64_t key, uint64_t first, float sigma) {
    size_t j = 0;
    if (first & 1) { row[0] = sigma * gauss_from_key(key, first); j = 1; }
    for (; j + 1 < cols; j += 2) {
        uint64_t h = splitmix64(key + ((first + j) >> 1));
        float u1 = (float)((h >> 40) + 1) * (1.0f / 16777216.0f);
        float u2 = (float)((h >> 8) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        float r = sqrtf(-2.0f * logf(u1));
        float th = 6.28318530717958647692f * u2;
        row[j] = sigma * (r * cosf(th));
        row[j + 1] = sigma * (r * sinf(th));
    }
    if (j < cols) row[j] = sigma * gauss_from_key(key, first + j);
}

static void synth_matrix(uint8_t* base, size_t off, size_t off_s, size_t rows, size_t cols,
                         int wbits, int group, float div, uint64_t seed, uint64_t stream,
                         float sigma) {
    uint64_t key = stream_key(seed, stream);
    const size_t rb = wbits == 4 ? cols / 2 : cols;
    const size_t nb = cols / (size_t)group;
    #pragma omp parallel
    {
        float* row = (float*)malloc(cols * sizeof(float));
        #pragma omp for schedule(static)
        for (long long r = 0; r < (long long)rows; r++) {
            gauss_row(row, cols, key, (uint64_t)r * cols, sigma);
            uint8_t* q = base + off + (size_t)r * rb;
            float* s = (float*)(base + off_s) + (size_t)r * nb;
            if (wbits == 4) qll_quantize_row_q4(row, (int)cols, group, div, q, s);
            else qll_quantize_row_q8(row, (int)cols, group, q, s);
        }
        free(row);
    }
}

int qll_synth_write(void* dst, const l2q_config* c, int wbits, int group,
                    float q4_divisor, uint64_t seed, float sigma) {
    qll_layout lay;
    if (qll_layout_compute(c, wbits, group, &lay)) return -1;
    uint8_t* out = (uint8_t*)dst;
    size_t hb = qll_write_header(out, c, wbits, group);
    uint8_t* base = out + hb;
    const size_t d = (size_t)c->dim, h = (size_t)c->hidden_dim, L = (size_t)c->n_layers;
    const size_t kv = d * (size_t)c->n_kv_heads / (size_t)c->n_heads;
    const size_t V = (size_t)c->vocab_size;
    {   /* embedding */
        float* emb = (float*)(base + lay.emb);
        uint64_t key = stream_key(seed, S_EMB);
        #pragma omp parallel for schedule(static)
        for (long long r = 0; r < (long long)V; r++) gauss_row(emb + (size_t)r * d, d, key, (uint64_t)r * d, sigma);
    }
    float* ra = (float*)(base + lay.rms_att);
    float* rf = (float*)(base + lay.rms_ffn);
    float* rl = (float*)(base + lay.rms_final);
    for (size_t i = 0; i < L * d; i++) { ra[i] = 1.0f; rf[i] = 1.0f; }
    for (size_t i = 0; i < d; i++) rl[i] = 1.0f;
    synth_matrix(base, lay.wq, lay.wq_s, L * d, d, wbits, group, q4_divisor, seed, S_WQ, sigma);
    synth_matrix(base, lay.wk, lay.wk_s, L * kv, d, wbits, group, q4_divisor, seed, S_WK, sigma);
    synth_matrix(base, lay.wv, lay.wv_s, L * kv, d, wbits, group, q4_divisor, seed, S_WV, sigma);
    synth_matrix(base, lay.wo, lay.wo_s, L * d, d, wbits, group, q4_divisor, seed, S_WO, sigma);
    synth_matrix(base, lay.w1, lay.w1_s, L * h, d, wbits, group, q4_divisor, seed, S_W1, sigma);
    synth_matrix(base, lay.w2, lay.w2_s, L * d, h, wbits, group, q4_divisor, seed, S_W2, sigma);
    synth_matrix(base, lay.w3, lay.w3_s, L * h, d, wbits, group, q4_divisor, seed, S_W3, sigma);
    synth_matrix(base, lay.wcls, lay.wcls_s, V, d, wbits, group, q4_divisor, seed, S_WCLS, sigma);
    return 0;
}

int qll_synth_write_file(const char* path, const l2q_config* c, int wbits, int group,
                         float q4_divisor, uint64_t seed, float sigma) {
    size_t n = qll_synth_size(c, wbits, group);
    if (!n) return -1;
    void* buf = malloc(n);
    if (!buf) return -1;
    int rc = qll_synth_write(buf, c, wbits, group, q4_divisor, seed, sigma);
    if (rc == 0) {
        FILE* f = fopen(path, "wb");
        if (!f) rc = -1;
        else {
            if (fwrite(buf, 1, n, f) != n) rc = -1;
            if (fclose(f) != 0) rc = -1;
        }
    }
    free(buf);
    return rc;
}
