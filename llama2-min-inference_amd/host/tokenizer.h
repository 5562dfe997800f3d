/* tokenizer.h - byte-pair tokenizer over the llama2.c `tokenizer.bin` format.
 *
 * File format (runq.c:444-465): u32 max_token_length, then for every id:
 * f32 score, i32 len, len bytes of piece text.
 * Behaviour follows runq.c:426-560: greedy highest-score pair merging, a
 * leading " " dummy-prefix token, UTF-8 code points looked up whole, unknown
 * bytes mapped to id byte+3, BOS = 1, EOS = 2.
 */
#ifndef L2Q_TOKENIZER_H
#define L2Q_TOKENIZER_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    char** pieces;           /* [vocab] NUL-terminated piece text */
    float* scores;           /* [vocab] merge priority            */
    int* by_text;            /* ids sorted by piece text          */
    int vocab_size;
    unsigned int max_token_length;
    char byte_text[256][2];  /* single-byte strings for <0xXX> pieces */
} l2q_tokenizer;

/* Load; returns 0 or -1 (message in err). */
int tok_load(l2q_tokenizer* t, const char* path, int vocab_size, char* err, int errlen);
void tok_free(l2q_tokenizer* t);

/* Id of an exact piece text, or -1. */
int tok_lookup(const l2q_tokenizer* t, const char* text);

/* Encode `text` into tokens (capacity strlen(text)+3), optional BOS/EOS.
 * Returns the number of tokens, or -1 if text is NULL. */
int tok_encode(l2q_tokenizer* t, const char* text, int bos, int eos, int* tokens);

/* Text of `token` following `prev` (leading space dropped after BOS,
 * "<0xXX>" pieces become the raw byte). */
const char* tok_decode(const l2q_tokenizer* t, int prev, int token);

/* Print a piece unless it is a single non-printable, non-space byte. */
void tok_print_piece(const char* piece);

/* Write a tokenizer file (used to synthesise one for random-id runs). */
int tok_write(const char* path, char* const* pieces, const float* scores, int n);

#ifdef __cplusplus
}
#endif
#endif
