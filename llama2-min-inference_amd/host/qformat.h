/* qformat.h - QLL8 / QLL4 checkpoint layout, reader and synthetic writer.
 *
 * File layout (little-endian), as written by tools/quantize_int8.py:11-37 and
 * tools/quantize_int4.py:9-26 and read by runq.c:230-278 and
 * v5-cuda-fused/run.cu:534-551:
 *
 *   u32 magic   0x384C4C51 "QLL8" | 0x344C4C51 "QLL4"
 *   u32 version 1 (QLL8, group 32) | 2 (QLL4, group 32) | 3 (either, group
 *               given by the u32 that follows the config; this build's
 *               extension for group sizes other than 32)
 *   i32 config[7]  dim, hidden_dim, n_layers, n_heads, n_kv_heads,
 *                  vocab_size (< 0: unshared classifier), seq_len
 *   [u32 group]    version 3 only
 *   fp32 emb [V][d], fp32 rms_att [L][d],
 *   Q wq [L*d][d], Q wk [L*kv][d], Q wv [L*kv][d], Q wo [L*d][d],
 *   fp32 rms_ffn [L][d],
 *   Q w1 [L*h][d], Q w2 [L*d][h], Q w3 [L*h][d],
 *   fp32 rms_final [d],
 *   Q wcls [V][d]
 *
 * where a Q matrix [rows][cols] is its weight bytes (QLL8: u8 = q + 128,
 * rows*cols bytes; QLL4: two nibbles per byte, rows*cols/2 bytes) followed
 * by fp32 scales [rows][cols/group].
 */
#ifndef L2Q_QFORMAT_H
#define L2Q_QFORMAT_H

#include <stddef.h>
#include <stdint.h>
#include "l2q.h"

#ifdef __cplusplus
extern "C" {
#endif

#define QLL8_MAGIC 0x384C4C51u
#define QLL4_MAGIC 0x344C4C51u
#define QLL_VERSION_Q8 1u
#define QLL_VERSION_Q4 2u
#define QLL_VERSION_GROUP 3u

/* Offsets (bytes from the start of the tensor section) of every tensor. */
typedef struct {
    size_t emb, rms_att;
    size_t wq, wq_s, wk, wk_s, wv, wv_s, wo, wo_s;
    size_t rms_ffn;
    size_t w1, w1_s, w2, w2_s, w3, w3_s;
    size_t rms_final;
    size_t wcls, wcls_s;
    size_t total;
} qll_layout;

/* Bytes of weights (not scales) of a rows x cols matrix at `wbits`. */
size_t qll_matrix_bytes(size_t rows, size_t cols, int wbits);

/* Compute tensor offsets; returns 0 on success, -1 on an inconsistent
 * config (non-divisible dims, group not dividing dim/hidden). */
int qll_layout_compute(const l2q_config* c, int wbits, int group, qll_layout* out);

/* Parsed header. */
typedef struct {
    l2q_config cfg;          /* vocab_size positive */
    int shared_weights;      /* 1 if the file's vocab_size was positive */
    int wbits;               /* 8 or 4 */
    int group;
    size_t header_bytes;     /* 36 or 40 */
} qll_header;

/* Parse a header from the first `n` bytes of a file.  Returns 0 or a
 * negative code and writes a message into err (if not NULL). */
int qll_parse_header(const void* data, size_t n, qll_header* h, char* err, size_t errlen);

/* Serialize a header; returns the number of bytes written (36 or 40). */
size_t qll_write_header(void* dst, const l2q_config* c, int wbits, int group);

/* A checkpoint opened read-only through mmap. */
typedef struct {
    qll_header h;
    const uint8_t* data;     /* whole file */
    size_t file_size;
    const uint8_t* weights;  /* data + header_bytes */
    size_t weights_bytes;
    int fd;
} qll_file;

int qll_open(const char* path, qll_file* f, char* err, size_t errlen);
void qll_close(qll_file* f);

/* ---------------- quantizers (offline path) ---------------------------- */

/* INT8 weights of one row: tools/quantize_int8.py:52-63.
 * s = amax/127 (1e-8 if 0), q = clip(rint(w/s), -127, 127), u8 = q + 128. */
void qll_quantize_row_q8(const float* w, int cols, int group, uint8_t* q, float* s);

/* INT4 weights of one row: tools/quantize_int4.py:38-51 with the scale
 * divisor as a parameter (8 in the reference tool, 7 in the 7B configs).
 * s = amax/div (1e-8 if 0), q = clip(rint(w/s), -8, 7), two's-complement
 * nibbles, low nibble = even column. */
void qll_quantize_row_q4(const float* w, int cols, int group, float divisor,
                         uint8_t* q, float* s);

/* ---------------- deterministic synthetic data ------------------------- */

/* Counter-based N(0,1) sample number `index` of stream `stream` under
 * `seed` (splitmix64 + Box-Muller in float); independent of thread count. */
float qll_gauss(uint64_t seed, uint64_t stream, uint64_t index);

/* Fill dst[0..n) with sigma * N(0,1) samples index0.. of a stream. */
void qll_gauss_fill(float* dst, size_t n, uint64_t seed, uint64_t stream,
                    uint64_t index0, float sigma);

/* Uniform integer in [lo, hi) for draw `index` of a stream. */
int qll_uniform_int(uint64_t seed, uint64_t stream, uint64_t index, int lo, int hi);

/* Size of a complete synthetic checkpoint file (header + tensors). */
size_t qll_synth_size(const l2q_config* c, int wbits, int group);

/* Write a complete random-init checkpoint into `dst` (qll_synth_size bytes):
 * every matrix and the embedding ~ N(0, sigma) from `seed`, RMSNorm weights
 * 1.0, unshared classifier, quantized with the offline quantizers above
 * (INT4 divisor `q4_divisor`).  The header is version 1/2 when group == 32
 * and version 3 otherwise.  Uses OpenMP over rows.  Returns 0 or -1. */
int qll_synth_write(void* dst, const l2q_config* c, int wbits, int group,
                    float q4_divisor, uint64_t seed, float sigma);

/* Same, into a file. */
int qll_synth_write_file(const char* path, const l2q_config* c, int wbits,
                         int group, float q4_divisor, uint64_t seed, float sigma);

#ifdef __cplusplus
}
#endif
#endif
