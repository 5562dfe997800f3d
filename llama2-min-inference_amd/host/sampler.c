/* sampler.c - see sampler.h. */
#include "sampler.h"

#include <math.h>
#include <stdlib.h>

int sampler_init(l2q_sampler* s, int vocab_size, float temperature, float topp,
                 unsigned long long seed) {
    s->vocab_size = vocab_size;
    s->temperature = temperature;
    s->topp = topp;
    s->rng_state = seed;
    s->scratch = (l2q_prob_index*)malloc((size_t)vocab_size * sizeof(l2q_prob_index));
    return s->scratch ? 0 : -1;
}

void sampler_free(l2q_sampler* s) {
    free(s->scratch);
    s->scratch = NULL;
}

int sampler_argmax(const float* v, int n) {
    int best = 0;
    float m = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > m) { m = v[i]; best = i; }
    return best;
}

void sampler_softmax(float* x, int n) {
    float m = x[0];
    for (int i = 1; i < n; i++) if (x[i] > m) m = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); sum += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

static unsigned int random_u32(unsigned long long* st) {
    *st ^= *st >> 12;
    *st ^= *st << 25;
    *st ^= *st >> 27;
    return (unsigned int)((*st * 0x2545F4914F6CDD1Dull) >> 32);
}

float sampler_random_f32(unsigned long long* st) {
    return (float)(random_u32(st) >> 8) / 16777216.0f;
}

/* Multinomial over an already-normalised distribution. */
static int sample_mult(const float* p, int n, float coin) {
    float cdf = 0.0f;
    for (int i = 0; i < n; i++) {
        cdf += p[i];
        if (coin < cdf) return i;
    }
    return n - 1;
}

/* Descending by probability; equal probabilities keep qsort's order. */
static int by_prob_desc(const void* a, const void* b) {
    float pa = ((const l2q_prob_index*)a)->prob, pb = ((const l2q_prob_index*)b)->prob;
    return pa > pb ? -1 : (pa < pb ? 1 : 0);
}

/* Nucleus sampling: candidates below (1-p)/(n-1) are dropped before the
 * sort, the smallest prefix whose mass exceeds p is kept, and the coin is
 * scaled to that prefix's mass. */
static int sample_topp(const float* p, int n, float topp, l2q_prob_index* buf, float coin) {
    int m = 0;
    const float cutoff = (1.0f - topp) / (float)(n - 1);
    for (int i = 0; i < n; i++)
        if (p[i] >= cutoff) { buf[m].index = i; buf[m].prob = p[i]; m++; }
    qsort(buf, (size_t)m, sizeof(l2q_prob_index), by_prob_desc);
    float mass = 0.0f;
    int last = m - 1;
    for (int i = 0; i < m; i++) {
        mass += buf[i].prob;
        if (mass > topp) { last = i; break; }
    }
    float r = coin * mass, cdf = 0.0f;
    for (int i = 0; i <= last; i++) {
        cdf += buf[i].prob;
        if (r < cdf) return buf[i].index;
    }
    return buf[last].index;
}

int sampler_sample(l2q_sampler* s, float* logits) {
    if (s->temperature == 0.0f) return sampler_argmax(logits, s->vocab_size);
    for (int i = 0; i < s->vocab_size; i++) logits[i] /= s->temperature;
    sampler_softmax(logits, s->vocab_size);
    float coin = sampler_random_f32(&s->rng_state);
    if (s->topp <= 0 || s->topp >= 1) return sample_mult(logits, s->vocab_size, coin);
    return sample_topp(logits, s->vocab_size, s->topp, s->scratch, coin);
}
