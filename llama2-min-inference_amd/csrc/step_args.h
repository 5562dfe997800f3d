// step_args.h - arguments of the one-kernel decode step (k_step, step.h),
// shared by the kernel and the engine that launches it.
#pragma once
#include <stdint.h>

#include "device.h"

namespace l2q {

constexpr int kStepCompute = 7;                              // compute waves (two waves per SIMD)
constexpr int kStepThreads = (kStepCompute + 1) * L2Q_WAVE;  // + the control wave
constexpr int kStepCThreads = kStepCompute * L2Q_WAVE;
constexpr int kStepStage = 32;       // staged outputs per wave and phase
constexpr int kStepAttnSlice = 16;   // output elements per attention workgroup item (kVDims)
constexpr int kStepPairsCap = 64;    // row pairs of a dim-wide GEMV per workgroup
constexpr int kStepPairsCapH = 8;    // row pairs of w2 per workgroup

// Barrier state (device memory, zeroed once): 8 group counters and the
// top counter on their own 64-byte lines, one release word per workgroup
// on its own line, the error word and the launch epoch.
struct StepSync {
    unsigned* grp;     // [8][16]
    unsigned* top;     // [16]
    unsigned* rel;     // [grid][16]
    unsigned* err;     // sticky: 1 = a barrier wait timed out
    unsigned* epoch;   // launches completed
};

struct StepArgs {
    const uint8_t *qkv_w, *wo_w, *w13_w, *w2_w, *wcls_w;
    const float *qkv_s, *wo_s, *w13_s, *w2_s, *wcls_s;
    const float *emb, *rms_att, *rms_ffn, *rms_final, *rope;
    float *xa, *xb, *q, *att, *wo_out, *hb, *ffn_out, *logits, *kcache, *vcache;
    const int* meta;
    float* dbg_x;      // optional: [L+1][d] residual stream (forward_debug)
    StepSync sync;
    int d, h, L, V, n_heads, n_kv, hs, kv, max_t;
    int rowb_d, rowb_h;
    int nbar;          // grid barriers per launch
};

__host__ __device__ constexpr int step_phases(int L) { return 5 * L + 1; }

}  // namespace l2q
