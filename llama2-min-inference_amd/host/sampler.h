/* sampler.h - next-token selection with the behaviour of runq.c:565-667:
 * greedy argmax at temperature 0, otherwise softmax(logits / T) and either
 * multinomial sampling or top-p (nucleus) sampling driven by a xorshift64*
 * generator, so that a given seed picks the same tokens as the reference. */
#ifndef L2Q_SAMPLER_H
#define L2Q_SAMPLER_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct { float prob; int index; } l2q_prob_index;

typedef struct {
    int vocab_size;
    float temperature;
    float topp;
    unsigned long long rng_state;
    l2q_prob_index* scratch;   /* [vocab_size] for top-p */
} l2q_sampler;

int sampler_init(l2q_sampler* s, int vocab_size, float temperature, float topp,
                 unsigned long long seed);
void sampler_free(l2q_sampler* s);

/* First index of the maximum (strict >), runq.c:578-585. */
int sampler_argmax(const float* v, int n);

/* In-place max-subtracted softmax, runq.c:307-318. */
void sampler_softmax(float* x, int n);

/* xorshift64* draw in [0,1), runq.c:642-650. */
float sampler_random_f32(unsigned long long* state);

/* Pick the next token; modifies `logits` when temperature > 0. */
int sampler_sample(l2q_sampler* s, float* logits);

#ifdef __cplusplus
}
#endif
#endif
