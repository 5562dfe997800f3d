// ops.hip - launchers and the op-level C ABI (see include/l2q.h).
#include <hip/hip_runtime.h>

#include <mutex>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kernels.h"
#include "prefill.h"
#include "launch.h"
#include "step.h"

namespace l2q {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return L2Q_ERR_HIP;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? L2Q_OK : hip_fail(e, what);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------------------
// GEMV dispatch.  NS = 1 KiB sweeps per row = ceil(cols*bits/8 / 1024).
constexpr int kMaxNS = 12;

bool gemv_shape_ok(int bits, int group, int rows, int cols) {
    if (bits != 4 && bits != 8) return false;
    if (group != 32 && group != 64) return false;
    if (rows <= 0 || cols <= 0 || cols % group) return false;
    return gemv_sweeps(bits, cols) <= kMaxNS;
}

// Workgroups of a persistent GEMV launch: the resident workgroups per CU
// (occupancy), at most `cap` per CU, times the CU count.
static int resident_blocks(const void* fn, int threads, size_t lds, int cap) {
    struct Entry { const void* fn; size_t lds; int dev; int blocks; };
    static thread_local Entry cache[64];
    static thread_local int used = 0;
    int dev = 0;
    (void)hipGetDevice(&dev);
    for (int i = 0; i < used; i++)
        if (cache[i].fn == fn && cache[i].lds == lds && cache[i].dev == dev) return cache[i].blocks;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess || per_cu < 1) per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
    (void)hipGetLastError();
    const int blocks = (per_cu < cap ? per_cu : cap) * cus;
    if (used < 64) cache[used++] = Entry{fn, lds, dev, blocks};
    return blocks;
}

// Raise a kernel's dynamic-LDS limit to `lds` bytes on the current device
// when it exceeds the default 64 KiB (gfx950 has 160 KiB per workgroup):
// once per (kernel, device, size) and calling thread (the attribute is
// idempotent, so threads need not share the record).
static int raise_lds_limit(const void* fn, size_t lds, const char* what) {
    if (lds <= 65536) return L2Q_OK;
    struct Entry { const void* fn; int dev; size_t lds; };
    static thread_local Entry done[64];
    static thread_local int used = 0;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, what);
    for (int i = 0; i < used; i++)
        if (done[i].fn == fn && done[i].dev == dev && done[i].lds >= lds) return L2Q_OK;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e, what);
    if (used < 64) done[used++] = Entry{fn, dev, lds};
    return L2Q_OK;
}

// One workgroup per CU (see gemv_waves).
constexpr int kGemvBlocksPerCu = 1;
constexpr size_t kGemvMaxLds = 160 * 1024;   // gfx950 LDS per workgroup

template <int BITS, int G, int NS, int PRO, int EPI, int W>
static int go_gemv_w(const GemvArgs& a, hipStream_t st) {
    constexpr int PR = gemv_unit_rows(NS, EPI);
    const size_t lds = gemv_lds_bytes(PRO, a.cols, G, BITS, PR, W);
    const void* fn = reinterpret_cast<const void*>(&k_gemv<BITS, G, NS, PRO, EPI, PR, W>);
    if (int rc = raise_lds_limit(fn, lds, "gemv: raising the LDS limit")) return rc;
    const int maxb = resident_blocks(fn, W * L2Q_WAVE, lds, kGemvBlocksPerCu);
    const int nunits = (a.rows + PR - 1) / PR;
    int blocks = (nunits + W - 1) / W;
    if (blocks > maxb) blocks = maxb;
    hipLaunchKernelGGL((k_gemv<BITS, G, NS, PRO, EPI, PR, W>), dim3(blocks), dim3(W * L2Q_WAVE), lds, st, a);
    return check_launch("gemv");
}

// Share of the grid's wave-rounds that carry a unit when `waves` waves
// (one workgroup per CU) deal `units` units round-robin: the last round
// runs only the remainder.
static double gemv_round_fill(long units, long waves) {
    const long rounds = (units + waves - 1) / waves;
    return rounds ? (double)units / (double)(rounds * waves) : 1.0;
}

template <int BITS, int G, int NS, int PRO, int EPI>
static int go_gemv(const GemvArgs& a, hipStream_t st) {
    if constexpr (NS == 2) {
        // rows of two sweeps: 11 waves per CU where that fills the last round
        // of units clearly better than 8 (the 7B w1|w3 GEMV: 11008 units,
        // 0.90 of the rounds busy with 8 waves, 0.98 with 11)
        constexpr int PR = gemv_unit_rows(NS, EPI);
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        const long units = (a.rows + PR - 1) / PR;
        if (units > (long)cus * gemv_waves(NS) &&
            gemv_round_fill(units, (long)cus * kGemvWavesWide) > gemv_round_fill(units, (long)cus * gemv_waves(NS)) + 0.05)
            return go_gemv_w<BITS, G, NS, PRO, EPI, kGemvWavesWide>(a, st);
    }
    return go_gemv_w<BITS, G, NS, PRO, EPI, gemv_waves(NS)>(a, st);
}

template <int BITS, int G, int PRO, int EPI>
static int gemv_by_t(const GemvArgs& a, hipStream_t st) {
    const int NS = gemv_sweeps(BITS, a.cols);
    switch (NS) {
        case 1: return go_gemv<BITS, G, 1, PRO, EPI>(a, st);
        case 2: return go_gemv<BITS, G, 2, PRO, EPI>(a, st);
        case 3: return go_gemv<BITS, G, 3, PRO, EPI>(a, st);
        case 4: return go_gemv<BITS, G, 4, PRO, EPI>(a, st);
    }
    if constexpr (PRO != kNorm) {   // the norm prologue only ever sees dim-long inputs
        switch (NS) {
            case 5: return go_gemv<BITS, G, 5, PRO, EPI>(a, st);
            case 6: return go_gemv<BITS, G, 6, PRO, EPI>(a, st);
            case 7: return go_gemv<BITS, G, 7, PRO, EPI>(a, st);
            case 8: return go_gemv<BITS, G, 8, PRO, EPI>(a, st);
            case 9: return go_gemv<BITS, G, 9, PRO, EPI>(a, st);
            case 10: return go_gemv<BITS, G, 10, PRO, EPI>(a, st);
            case 11: return go_gemv<BITS, G, 11, PRO, EPI>(a, st);
            case 12: return go_gemv<BITS, G, 12, PRO, EPI>(a, st);
        }
    }
    set_error("gemv: %d columns exceed the supported range for this prologue", a.cols);
    return L2Q_ERR_ARG;
}

template <int PRO, int EPI>
static int gemv_by_bits(int bits, int group, const GemvArgs& a, hipStream_t st) {
    if (bits == 4) return group == 32 ? gemv_by_t<4, 32, PRO, EPI>(a, st) : gemv_by_t<4, 64, PRO, EPI>(a, st);
    return group == 32 ? gemv_by_t<8, 32, PRO, EPI>(a, st) : gemv_by_t<8, 64, PRO, EPI>(a, st);
}

int launch_gemv_fused(int bits, int group, int pro, int epi, const GemvArgs& a, hipStream_t st) {
    if (!gemv_shape_ok(bits, group, a.rows, a.cols)) {
        set_error("gemv: unsupported shape bits=%d group=%d rows=%d cols=%d", bits, group, a.rows, a.cols);
        return L2Q_ERR_ARG;
    }
    if (!a.w || !a.ws || !aligned16(a.w)) { set_error("gemv: weights must be non-null and 16-byte aligned"); return L2Q_ERR_ARG; }
    if (pro == kPreq && (!a.xq || !a.xs || !aligned16(a.xq))) {
        set_error("gemv: activations must be non-null and 16-byte aligned");
        return L2Q_ERR_ARG;
    }
    if (pro != kPreq && !a.x_in && !(pro == kNorm && a.emb)) { set_error("gemv: null prologue input"); return L2Q_ERR_ARG; }
    if (pro == kNorm && (!a.norm_w || (a.emb && !a.meta))) { set_error("gemv: null norm weight / meta"); return L2Q_ERR_ARG; }
    if (gemv_lds_bytes(pro, a.cols, group, bits, 2) > kGemvMaxLds) {
        set_error("gemv: cols=%d needs too much LDS", a.cols);
        return L2Q_ERR_ARG;
    }
    if (pro == kNorm && gemv_sweeps(bits, a.cols) > 4) {
        set_error("gemv: the norm prologue supports rows of at most 4 KiB");
        return L2Q_ERR_ARG;
    }
    if (epi == kRopeKV && (!a.meta || !a.rope || !a.kcache || !a.vcache || a.hs <= 0 || a.hs % 2 || a.dim % a.hs ||
                           a.kv_dim % a.hs || a.rows != a.dim + 2 * a.kv_dim || !a.out || a.max_t <= 0 ||
                           a.hs > kAttnMaxHs || a.rows >= 65536)) {
        set_error("gemv: bad RoPE/KV epilogue arguments");
        return L2Q_ERR_ARG;
    }
    if (!a.out) { set_error("gemv: null output"); return L2Q_ERR_ARG; }
    if (epi == kSwiglu && a.rows % 2) { set_error("gemv: the SwiGLU epilogue needs (w1, w3) row pairs"); return L2Q_ERR_ARG; }
    if (pro == kPreq && epi == kStore) return gemv_by_bits<kPreq, kStore>(bits, group, a, st);
    if (pro == kQuant && epi == kStore) return gemv_by_bits<kQuant, kStore>(bits, group, a, st);
    if (pro == kNorm && epi == kStore) return gemv_by_bits<kNorm, kStore>(bits, group, a, st);
    if (pro == kNorm && epi == kRopeKV) return gemv_by_bits<kNorm, kRopeKV>(bits, group, a, st);
    if (pro == kNorm && epi == kSwiglu) return gemv_by_bits<kNorm, kSwiglu>(bits, group, a, st);
    set_error("gemv: unsupported prologue/epilogue combination %d/%d", pro, epi);
    return L2Q_ERR_ARG;
}

int launch_gemv(int bits, int group, const GemvArgs& a, hipStream_t st) {
    return launch_gemv_fused(bits, group, kPreq, kStore, a, st);
}

// ---------------------------------------------------------------------------

// The optional prefill operand of a producer: checked, or all null.
static int pf_operand(const PfOperand* pf, int8_t* xq, const float* xs, int K, int T, PfOperand* out,
                      const char* what) {
    *out = PfOperand{nullptr, nullptr, 8, 1, 1};
    if (!pf) {
        if (!xq || !xs) { set_error("%s: no output", what); return L2Q_ERR_ARG; }
        return L2Q_OK;
    }
    if (!pf->xqp || !pf->rec || (pf->bits != 4 && pf->bits != 8) || pf->K != K || pf->T != T) {
        set_error("%s: bad prefill operand (bits=%d K=%d T=%d for %d x %d)", what, pf->bits, pf->K, pf->T, T, K);
        return L2Q_ERR_ARG;
    }
    *out = *pf;
    return L2Q_OK;
}

int launch_quantize(const float* x, int n, int group, int8_t* xq, float* xs, hipStream_t st, const PfOperand* pf) {
    if (n <= 0 || (group != 32 && group != 64) || n % group) { set_error("quantize: bad n=%d group=%d", n, group); return L2Q_ERR_ARG; }
    if (pf && (pf->K <= 0 || pf->K % group || n % pf->K)) { set_error("quantize: prefill operand rows of %d", pf->K); return L2Q_ERR_ARG; }
    PfOperand po;
    if (int rc = pf_operand(pf, xq, xs, pf ? pf->K : n, pf ? n / pf->K : 1, &po, "quantize")) return rc;
    const int blocks = (n + 255) / 256;
    if (group == 32) hipLaunchKernelGGL(k_quantize<32>, dim3(blocks), dim3(256), 0, st, x, n, xq, xs, po);
    else hipLaunchKernelGGL(k_quantize<64>, dim3(blocks), dim3(256), 0, st, x, n, xq, xs, po);
    return check_launch("quantize");
}

int launch_rmsnorm_quant(const float* x, const float* emb, const int* meta, const float* resid, float* xout,
                         const float* w, int n, int group, int8_t* xq, float* xs, hipStream_t st, int T,
                         const PfOperand* pf) {
    if (n <= 0 || n > kNormThreads * kNormMaxPer || (group != 32 && group != 64) || n % group || T < 1 ||
        (T > 1 && emb)) {
        set_error("rmsnorm_quant: bad n=%d group=%d T=%d", n, group, T);
        return L2Q_ERR_ARG;
    }
    if (pf) {
        // the GEMM operand of a prefill batch: float4 chunks, each token on kPfNormSplit workgroups
        PfOperand po;
        if (int rc = pf_operand(pf, nullptr, nullptr, n, T, &po, "rmsnorm_quant")) return rc;
        if (emb || xq || xs || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(resid) % 16 ||
            reinterpret_cast<uintptr_t>(xout) % 16 || reinterpret_cast<uintptr_t>(w) % 16) {
            set_error("rmsnorm_quant: the GEMM operand form takes 16-byte aligned x, resid, xout, w and no other output");
            return L2Q_ERR_ARG;
        }
        const dim3 grid(kPfNormSplit, (unsigned)T);
        if (group == 32)
            hipLaunchKernelGGL(k_pf_rmsnorm_quant<32>, grid, dim3(kPfNormThreads), 0, st, x, resid, xout, w, n, po);
        else
            hipLaunchKernelGGL(k_pf_rmsnorm_quant<64>, grid, dim3(kPfNormThreads), 0, st, x, resid, xout, w, n, po);
        return check_launch("prefill_rmsnorm_quant");
    }
    if (!xq || !xs) { set_error("rmsnorm_quant: no output"); return L2Q_ERR_ARG; }
    if (group == 32)
        hipLaunchKernelGGL(k_rmsnorm_quant<32>, dim3(T), dim3(kNormThreads), 0, st, x, emb, meta, resid, xout, w, n, xq, xs);
    else
        hipLaunchKernelGGL(k_rmsnorm_quant<64>, dim3(T), dim3(kNormThreads), 0, st, x, emb, meta, resid, xout, w, n, xq, xs);
    return check_launch("rmsnorm_quant");
}

int launch_swiglu_quant(const float* hb, const float* hb2, int n, int group, int8_t* xq, float* xs, float* gout,
                        hipStream_t st) {
    if (n <= 0 || (group != 32 && group != 64) || n % group) { set_error("swiglu_quant: bad n=%d group=%d", n, group); return L2Q_ERR_ARG; }
    const int blocks = (n + 255) / 256;
    if (group == 32) hipLaunchKernelGGL(k_swiglu_quant<32>, dim3(blocks), dim3(256), 0, st, hb, hb2, n, xq, xs, gout);
    else hipLaunchKernelGGL(k_swiglu_quant<64>, dim3(blocks), dim3(256), 0, st, hb, hb2, n, xq, xs, gout);
    return check_launch("swiglu_quant");
}

int launch_rope_kv_append(float* q, const float* k, const float* v, float* kcache, float* vcache, const float* rope,
                          const int* meta, int pos, int dim, int kv_dim, int hs, int max_t, hipStream_t st, int T,
                          int stride, int k_il) {
    if (hs <= 0 || hs % 2 || (k_il && hs % 4) || dim % hs || kv_dim % hs || kv_dim > dim || max_t <= 0 || T < 1 ||
        (!meta && (pos < 0 || pos + T > max_t)) || (meta && T > 1)) {
        set_error("rope_kv_append: bad shape dim=%d kv_dim=%d hs=%d pos=%d T=%d max_t=%d", dim, kv_dim, hs, pos, T,
                  max_t);
        return L2Q_ERR_ARG;
    }
    const int pairs = dim / 2;
    hipLaunchKernelGGL(k_rope_kv_append, dim3((pairs + 255) / 256, T), dim3(256), 0, st, q, k, v, kcache, vcache,
                       rope, meta, pos, dim, kv_dim, hs, max_t, stride, k_il);
    return check_launch("rope_kv_append");
}

bool attention_shape_ok(int n_heads, int n_kv_heads, int hs) {
    return n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && hs > 0 && hs % 4 == 0 &&
           hs <= kAttnMaxHs;
}

int launch_attention_split(const float* q, const float* kcache, const float* vcache, float* out, float* part_o,
                           float* part_ml, int S, const int* meta, int pos, int n_heads, int n_kv_heads, int hs,
                           int max_t, hipStream_t st) {
    if (!attention_shape_ok(n_heads, n_kv_heads, hs) || S <= 0 || max_t <= 0 ||
        (!meta && (pos < 0 || pos >= max_t))) {
        set_error("attention: bad shape heads=%d kv_heads=%d hs=%d S=%d pos=%d max_t=%d", n_heads, n_kv_heads, hs, S,
                  pos, max_t);
        return L2Q_ERR_ARG;
    }
    const int nmax = meta ? max_t : pos + 1;   // a captured graph covers every position
    const size_t lds = attn_lds_bytes((nmax + S - 1) / S, hs);
    if (lds > 65536) {
        set_error("attention: %d positions per split exceed the LDS budget", (nmax + S - 1) / S);
        return L2Q_ERR_ARG;
    }
    hipLaunchKernelGGL(k_attn_partial, dim3(n_heads, S), dim3(kAttnThreads), lds, st, q, kcache, vcache, part_o,
                       part_ml, meta, pos, n_heads, n_heads / n_kv_heads, hs, max_t);
    int rc = check_launch("attention_partial");
    if (rc) return rc;
    hipLaunchKernelGGL(k_attn_combine, dim3(n_heads), dim3(hs < 256 ? hs : 256), 0, st, part_o, part_ml, out, S, hs);
    return check_launch("attention_combine");
}

template <int HS, int KIL>
static int go_attn_fused_l(const float* q, const float* kcache, const float* vcache, float* out, const int* meta,
                           int pos, int kv_mul, int n_heads, int max_t, hipStream_t st) {
    const size_t lds = attn_fused_lds_bytes(max_t, HS);
    const void* fn = reinterpret_cast<const void*>(&k_attn_fused<HS, KIL>);
    if (int rc = raise_lds_limit(fn, lds, "attention: raising the LDS limit")) return rc;
    hipLaunchKernelGGL((k_attn_fused<HS, KIL>), dim3(n_heads * (HS / kVDims)), dim3(kAfThreads), lds, st, q, kcache,
                       vcache, out, meta, pos, kv_mul, n_heads, max_t);
    return check_launch("attention_fused");
}

template <int HS>
static int go_attn_fused(const float* q, const float* kcache, const float* vcache, float* out, const int* meta,
                         int pos, int kv_mul, int n_heads, int max_t, int k_il, hipStream_t st) {
    return k_il ? go_attn_fused_l<HS, 1>(q, kcache, vcache, out, meta, pos, kv_mul, n_heads, max_t, st)
                : go_attn_fused_l<HS, 0>(q, kcache, vcache, out, meta, pos, kv_mul, n_heads, max_t, st);
}

bool attention_fused_ok(int hs) { return hs == 48 || hs == 64 || hs == 128; }

int attention_fused_max() {
    static const int v = [] {
        const char* s = getenv("L2Q_ATTN_FUSED_MAX");
        return s ? atoi(s) : kAfDefaultMax;
    }();
    return v;
}

int attention_exact_max() { return kScorePer * kAttnThreads; }

bool attention_exact_ok(int max_t) {
    return max_t <= kScorePer * kAttnThreads && attn_v_lds_bytes(max_t) <= 65536;
}

bool attention_flash_ok(int hs) { return hs == 48 || hs == 64 || hs == 128; }

int attention_flash_splits(int n_heads, int max_t, int ncu) {
    int S = (2 * (ncu > 0 ? ncu : 256) + n_heads - 1) / n_heads;   // about two workgroups per CU
    const int need = (max_t + kFlMaxC - 1) / kFlMaxC;
    if (S < need) S = need;
    return S < 1 ? 1 : (S > kFlMaxSplits ? kFlMaxSplits : S);
}

size_t attention_flash_part_floats(int n_heads, int S, int hs) { return (size_t)n_heads * S * (hs + 2); }

template <int HS>
static int go_attn_flash(const float* q, const float* kcache, const float* vcache, float* out, float* part,
                         unsigned* cnt, int S, const int* meta, int pos, int n_heads, int kv_mul, int max_t, int k_il,
                         hipStream_t st) {
    if (k_il)
        hipLaunchKernelGGL((k_attn_flash<HS, 1>), dim3(n_heads, S), dim3(kFlThreads), 0, st, q, kcache, vcache, out,
                           part, cnt, meta, pos, kv_mul, max_t);
    else
        hipLaunchKernelGGL((k_attn_flash<HS, 0>), dim3(n_heads, S), dim3(kFlThreads), 0, st, q, kcache, vcache, out,
                           part, cnt, meta, pos, kv_mul, max_t);
    return check_launch("attention_flash");
}

int launch_attention_flash(const float* q, const float* kcache, const float* vcache, float* out, float* part,
                           unsigned* cnt, int S, const int* meta, int pos, int n_heads, int n_kv_heads, int hs,
                           int max_t, int k_il, hipStream_t st) {
    // positions a launch may cover: any of the cache's under a captured graph
    const int nmax = meta ? max_t : pos + 1;
    if (!attention_shape_ok(n_heads, n_kv_heads, hs) || !attention_flash_ok(hs) || S <= 0 || S > kFlMaxSplits ||
        max_t <= 0 || (!meta && (pos < 0 || pos >= max_t)) || (nmax + S - 1) / S > kFlMaxC || !part || !cnt) {
        set_error("attention_flash: bad shape heads=%d kv_heads=%d hs=%d S=%d pos=%d max_t=%d", n_heads, n_kv_heads,
                  hs, S, pos, max_t);
        return L2Q_ERR_ARG;
    }
    const int kv_mul = n_heads / n_kv_heads;
    switch (hs) {
        case 48: return go_attn_flash<48>(q, kcache, vcache, out, part, cnt, S, meta, pos, n_heads, kv_mul, max_t, k_il, st);
        case 64: return go_attn_flash<64>(q, kcache, vcache, out, part, cnt, S, meta, pos, n_heads, kv_mul, max_t, k_il, st);
        default: return go_attn_flash<128>(q, kcache, vcache, out, part, cnt, S, meta, pos, n_heads, kv_mul, max_t, k_il, st);
    }
}

// The batched scores kernel (T > 1 queries at positions pos..pos+T-1).
static int launch_attention_scores_b(const float* q, const float* kcache, float* scores, int pos, int T, int kv_mul,
                                     int n_heads, int hs, int max_t, int q_stride, int k_il, hipStream_t st) {
    const int nk = pos + T;
    const size_t lds = attn_scores_b_lds_bytes(hs);
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(&k_attn_scores_b), lds,
                                 "attention: raising the LDS limit"))
        return rc;
    hipLaunchKernelGGL(k_attn_scores_b, dim3(n_heads, (nk + kSbKeys - 1) / kSbKeys, (T + kSbQueries - 1) / kSbQueries),
                       dim3(kSbThreads), lds, st, q, kcache, scores, pos, T, kv_mul, n_heads, hs, max_t, q_stride, k_il);
    return check_launch("attention_scores_b");
}

int launch_attention_exact(const float* q, const float* kcache, const float* vcache, float* out, float* scores,
                           int S, const int* meta, int pos, int n_heads, int n_kv_heads, int hs, int max_t,
                           hipStream_t st, int T, int q_stride, int fused, int k_il) {
    (void)S;
    if (!attention_shape_ok(n_heads, n_kv_heads, hs) || max_t <= 0 || !attention_exact_ok(max_t) || T < 1 ||
        (!meta && (pos < 0 || pos + T > max_t)) || (meta && T > 1)) {
        set_error("attention: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d", n_heads, n_kv_heads, hs, pos,
                  max_t);
        return L2Q_ERR_ARG;
    }
    const int kv_mul = n_heads / n_kv_heads;
    const bool one = T == 1 && attention_fused_ok(hs) &&
                     (fused == 1 || (fused == -1 && !meta && pos + 1 <= attention_fused_max()));
    if (one) {   // one query: the single-kernel form (same operations, same order)
        switch (hs) {
            case 48: return go_attn_fused<48>(q, kcache, vcache, out, meta, pos, kv_mul, n_heads, max_t, k_il, st);
            case 64: return go_attn_fused<64>(q, kcache, vcache, out, meta, pos, kv_mul, n_heads, max_t, k_il, st);
            case 128: return go_attn_fused<128>(q, kcache, vcache, out, meta, pos, kv_mul, n_heads, max_t, k_il, st);
        }
    }
    if (T > 1 && !meta) {
        // a batch of queries: K and V rows shared over the queries (same
        // operations, same order as the per-query kernels below)
        int rc = launch_attention_scores_b(q, kcache, scores, pos, T, kv_mul, n_heads, hs, max_t, q_stride, k_il, st);
        if (rc) return rc;
        hipLaunchKernelGGL(k_attn_softmax_b, dim3(T, n_heads), dim3(kSmThreads), attn_softmax_b_lds_bytes(pos + T), st,
                           scores, pos, n_heads, max_t, pos + T);
        if ((rc = check_launch("attention_softmax_b"))) return rc;
        hipLaunchKernelGGL(k_attn_pv_b, dim3(n_heads, (hs + kVDims - 1) / kVDims, (T + kPvQueries - 1) / kPvQueries),
                           dim3(kPvThreads), 0, st, scores, vcache, out, pos, T, kv_mul, n_heads, hs, max_t);
        return check_launch("attention_pv_b");
    }
    // persistent score waves over (head, tile) items; a captured graph covers
    // every position the cache can hold, items past pos are not visited
    const int items = n_heads * ((meta ? max_t : pos + T) + kScoreTile - 1) / kScoreTile;
    const int grid = items < kScoreGridMax ? items : kScoreGridMax;
    hipLaunchKernelGGL(k_attn_scores, dim3(grid, T), dim3(kScoreThreads), attn_scores_lds_bytes(hs), st, q, kcache,
                       scores, meta, pos, kv_mul, n_heads, hs, max_t, q_stride, k_il);
    int rc = check_launch("attention_scores");
    if (rc) return rc;
    hipLaunchKernelGGL(k_attn_softmax_v, dim3(n_heads, (hs + kVDims - 1) / kVDims, T), dim3(kAttnThreads),
                       attn_v_lds_bytes(max_t), st, scores, vcache, out, meta, pos, kv_mul, hs, max_t);
    return check_launch("attention_softmax_v");
}

int launch_attention_prefill(const float* q, const float* kcache, const float* vcache, float* out, float* scores,
                             int pos, int n_heads, int n_kv_heads, int hs, int max_t, hipStream_t st, int T,
                             int q_stride, int k_il, int group, const PfOperand* pf) {
    const bool fuse = T > 1 && (hs == 64 || hs == 128) && hs % group == 0 && pos + T <= kPqMaxKeys &&
                      attention_shape_ok(n_heads, n_kv_heads, hs) && pos >= 0 && pos + T <= max_t &&
                      attention_exact_ok(max_t) && (group == 32 || group == 64);
    if (!fuse) {
        int rc = launch_attention_exact(q, kcache, vcache, out, scores, 0, nullptr, pos, n_heads, n_kv_heads, hs,
                                        max_t, st, T, q_stride, -1, k_il);
        if (rc || !pf) return rc;
        return launch_quantize(out, T * n_heads * hs, group, nullptr, nullptr, st, pf);
    }
    if (pf && (!pf->xqp || !pf->rec || (pf->bits != 4 && pf->bits != 8) || pf->K != n_heads * hs || pf->T != T)) {
        set_error("attention prefill: bad GEMM operand");
        return L2Q_ERR_ARG;
    }
    const int kv_mul = n_heads / n_kv_heads;
    const PfOperand po = pf ? *pf : PfOperand{nullptr, nullptr, 8, 1, 1};
    const dim3 grid((unsigned)n_heads, (unsigned)((T + kPqQueries - 1) / kPqQueries));
#define L2Q_PQ(HS_, G_)                                                                                         \
    hipLaunchKernelGGL((k_attn_pf_b<HS_, G_>), grid, dim3(kPqQueries * HS_ / 4), 0, st, q, q_stride, kcache, k_il, \
                       vcache, out, pos, T, kv_mul, n_heads, max_t, po)
    if (hs == 128) {
        if (group == 64) L2Q_PQ(128, 64);
        else L2Q_PQ(128, 32);
    } else {
        if (group == 64) L2Q_PQ(64, 64);
        else L2Q_PQ(64, 32);
    }
#undef L2Q_PQ
    return check_launch("attention_pf_b");
}

bool kv8_shape_ok(int n_heads, int n_kv_heads, int hs, int max_t) {
    return attention_shape_ok(n_heads, n_kv_heads, hs) && hs % 16 == 0 && max_t > 0 && max_t <= 8192;
}

int launch_kv8_append(const float* k, const float* v, int8_t* k8, int8_t* v8, float* ks, float* vs,
                      const float* rope, const int* meta, int pos, int n_kv_heads, int hs, int max_t,
                      hipStream_t st, int nrows, int src_rows) {
    if (!kv8_shape_ok(n_kv_heads, n_kv_heads, hs, max_t) || (!meta && (pos < 0 || pos >= max_t)) || !k || !v ||
        !k8 || !v8 || !ks || !vs || nrows < 1 || nrows > 65535 || src_rows < nrows ||
        (nrows > 1 && (meta || pos + nrows > max_t))) {
        set_error("kv8 append: bad arguments kv_heads=%d hs=%d pos=%d max_t=%d rows=%d", n_kv_heads, hs, pos, max_t,
                  nrows);
        return L2Q_ERR_ARG;
    }
    hipLaunchKernelGGL(k_kv8_append, dim3(n_kv_heads, 2, nrows), dim3(L2Q_WAVE), 0, st, k, v, k8, v8, ks, vs, rope,
                       meta, pos, hs, max_t, src_rows);
    return check_launch("kv8_append");
}

int launch_attention_kv8(const float* q, int8_t* k8, int8_t* v8, float* ks, float* vs, float* out, float* scores,
                         const int* meta, int pos, int n_heads, int n_kv_heads, int hs, int max_t, hipStream_t st,
                         const float* kst, const float* vst, int nq, int q_stride, int out_stride) {
    if (!kv8_shape_ok(n_heads, n_kv_heads, hs, max_t) || (!meta && (pos < 0 || pos >= max_t)) ||
        (!kst != !vst) || nq < 1 || nq > 65535 || (nq > 1 && (kst || meta || pos + nq > max_t))) {
        set_error("attention kv8: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d", n_heads, n_kv_heads, hs,
                  pos, max_t);
        return L2Q_ERR_ARG;
    }
    (void)scores;
    const int kv_mul = n_heads / n_kv_heads;
    const size_t lds = attn8_fused_lds_bytes(max_t);
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(&k_attn8_fused), lds,
                                 "attention kv8: raising the LDS limit"))
        return rc;
    hipLaunchKernelGGL(k_attn8_fused, dim3(n_heads, nq), dim3(kA8Threads), lds, st, q, kst, vst, k8, v8, ks, vs, out,
                       meta, pos, kv_mul, hs, max_t, q_stride, out_stride);
    return check_launch("attention_kv8");
}

int launch_attention_kv8_split(const float* q, const float* kst, const float* vst, int8_t* k8, int8_t* v8,
                               float* ks, float* vs, float* out, float* part, unsigned* cnt, int S, const int* meta,
                               int pos, int n_heads, int n_kv_heads, int hs, int max_t, hipStream_t st, int nq,
                               int q_stride, int out_stride) {
    // positions a launch may cover: any of the cache's under a captured graph
    const int nmax = meta ? max_t : pos + nq;
    if (!kv8_shape_ok(n_heads, n_kv_heads, hs, max_t) || (!meta && (pos < 0 || pos >= max_t)) || (!kst != !vst) ||
        S < 1 || S > kFlMaxSplits || (nmax + S - 1) / S > kA8sMaxC || !part || !cnt || nq < 1 || nq > 65535 ||
        (nq > 1 && (kst || meta || pos + nq > max_t))) {
        set_error("attention kv8 split: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d S=%d", n_heads,
                  n_kv_heads, hs, pos, max_t, S);
        return L2Q_ERR_ARG;
    }
    const size_t lds = attn8_split_lds_bytes(S, hs);
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(&k_attn8_split), lds,
                                 "attention kv8 split: raising the LDS limit"))
        return rc;
    hipLaunchKernelGGL(k_attn8_split, dim3(n_heads, S, nq), dim3(kA8sThreads), lds, st, q, kst, vst, k8, v8, ks, vs,
                       out, part, cnt, meta, pos, n_heads / n_kv_heads, hs, max_t, q_stride, out_stride);
    return check_launch("attention_kv8_split");
}

// ---------------------------------------------------------------------------
// batched prefill

int launch_pf_prep(int bits, int group, const int8_t* xq, const float* xs, int K, int T, int8_t* xqp, PfRecord* rec,
                   hipStream_t st) {
    if (T < 1 || K <= 0 || (group != 32 && group != 64) || K % group || (bits != 4 && bits != 8)) {
        set_error("prefill prep: bad K=%d T=%d group=%d bits=%d", K, T, group, bits);
        return L2Q_ERR_ARG;
    }
    const int n = T * (K / group), blocks = (n + 255) / 256;
    if (bits == 4 && group == 64) hipLaunchKernelGGL((k_pf_prep<4, 64>), dim3(blocks), dim3(256), 0, st, xq, xs, K, T, xqp, rec);
    if (bits == 4 && group == 32) hipLaunchKernelGGL((k_pf_prep<4, 32>), dim3(blocks), dim3(256), 0, st, xq, xs, K, T, xqp, rec);
    if (bits == 8 && group == 64) hipLaunchKernelGGL((k_pf_prep<8, 64>), dim3(blocks), dim3(256), 0, st, xq, xs, K, T, xqp, rec);
    if (bits == 8 && group == 32) hipLaunchKernelGGL((k_pf_prep<8, 32>), dim3(blocks), dim3(256), 0, st, xq, xs, K, T, xqp, rec);
    return check_launch("prefill_prep");
}

namespace {

// One workgroup shape of the batched GEMM: waves WR x WT of RTW x TPW
// 16x16 tiles, SC columns per step.
template <int B_, int G_, int RTW, int TPW, int WR, int WT, int SC, int NST, bool PIPE, int EPI>
void pf3_launch(const uint8_t* w, const float* ws, int rows, int cols, const int8_t* xqp, const PfRecord* rec, int T,
                float* out, int ldo, const PfRope& rp, hipStream_t st, const PfOperand& so = PfOperand{}) {
    using P = Pf3<B_, G_, RTW, TPW, WR, WT, SC>;
    const dim3 grid((unsigned)((rows + P::RT - 1) / P::RT), (unsigned)((T + P::TT - 1) / P::TT));
    hipLaunchKernelGGL((k_pf_gemm3<B_, G_, RTW, TPW, WR, WT, SC, NST, PIPE, EPI>), grid, dim3(P::NT), 0, st, w, ws,
                       rows, cols, xqp, rec, T, out, ldo, rp, so);
}

// The w1|w3 GEMM with the SwiGLU + Q8 stores (EPI 2): 2G-row workgroups,
// one quantization group of the hidden vector each (8 waves: 4 x 2 of 32 x 16
// for G64, 2 x 4 for G32; the 128-row tile measures as fast as the 64-row
// one on w1|w3).
template <int B_, int G_>
void pf3_swiglu(const uint8_t* w, const float* ws, int rows, int cols, const int8_t* xqp, const PfRecord* rec, int T,
                const PfOperand& so, hipStream_t st) {
    if constexpr (G_ == 64)
        pf3_launch<B_, G_, 2, 1, 4, 2, 2 * G_, 3, false, 2>(w, ws, rows, cols, xqp, rec, T, nullptr, rows, PfRope{}, st, so);
    else
        pf3_launch<B_, G_, 2, 1, 2, 4, 2 * G_, 3, false, 2>(w, ws, rows, cols, xqp, rec, T, nullptr, rows, PfRope{}, st, so);
}

// The two workgroup shapes of the batched GEMM (16x16 MFMA tiles; SC =
// columns per step, a multiple of the group):
//   wide   64 rows x 64 tokens, 8 waves (2 x 4) of 32 x 16, two groups per step
//   small  32 rows x 32 tokens, 4 waves (2 x 2) of 16 x 16, four groups per step
// A step's fixed costs (barrier, DMA wait, LDS and MFMA latency) are spread
// over the waves resident on a SIMD and over the work of the step: the
// wide tile does less LDS traffic and unpacking per output, the small tile
// with long steps keeps every SIMD busy when there are few rows (the
// ordered fold cannot split the columns).  Measured on MI355X at the 7B
// shapes, T = 127: qkv and w1|w3 wide, wo and w2 small (other shapes
// tried: 64 x 64 with 4 waves of 32 x 32, 32 x 64 with 16 x 32, 8-wave
// 64 x 128 and 128 x 64, one to eight groups per step, 3 to 5 stages).
// Workgroup tiles (rows x tokens): wide 64 x 64 (8 waves of 32 x 16) when
// its grid gives every CU two workgroups; narrow 64 x 32 (4 waves of 16 x 32:
// a wave's unpacked weights serve two token tiles, and the finer grid fills
// the CUs more evenly: the 7B qkv at 127 tokens 32.8 vs 35.3 us); then mid
// 64 x 32 (8 waves of 16 x 16) and small 32 x 32 (4 waves), the largest that
// still gives every CU a workgroup (fewer re-reads of activations and weights).
enum PfShape { kPfWide, kPfNarrow, kPfMid, kPfSmall };

template <int B_, int G_, int EPI>
void pf3_shape(PfShape shp, const uint8_t* w, const float* ws, int rows, int cols, const int8_t* xqp,
               const PfRecord* rec, int T, float* out, int ldo, const PfRope& rp, hipStream_t st) {
    if (shp == kPfWide)
        pf3_launch<B_, G_, 2, 1, 2, 4, 2 * G_, 3, false, EPI>(w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
    else if (shp == kPfNarrow)
        pf3_launch<B_, G_, 1, 2, 4, 1, 2 * G_, 3, false, EPI>(w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
    else if (shp == kPfMid)
        pf3_launch<B_, G_, 1, 1, 4, 2, 4 * G_, 4, false, EPI>(w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
    else
        pf3_launch<B_, G_, 1, 1, 2, 2, 4 * G_, 4, false, EPI>(w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
}

template <int EPI>
void pf3_bits(int bits, int group, PfShape shp, const uint8_t* w, const float* ws, int rows, int cols,
              const int8_t* xqp, const PfRecord* rec, int T, float* out, int ldo, const PfRope& rp, hipStream_t st) {
    if (bits == 4 && group == 64) pf3_shape<4, 64, EPI>(shp, w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
    if (bits == 4 && group == 32) pf3_shape<4, 32, EPI>(shp, w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
    if (bits == 8 && group == 64) pf3_shape<8, 64, EPI>(shp, w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
    if (bits == 8 && group == 32) pf3_shape<8, 32, EPI>(shp, w, ws, rows, cols, xqp, rec, T, out, ldo, rp, st);
}

}  // namespace

int launch_pf_gemm(int bits, int group, const void* w, const float* ws, int rows, int cols, const int8_t* xqp,
                   const PfRecord* rec, int T, float* out, int ldo, hipStream_t st, const PfRope* rope,
                   const PfOperand* swiglu) {
    if (T < 1 || rows < 1 || cols <= 0 || (group != 32 && group != 64) || cols % group || (bits != 4 && bits != 8) ||
        cols % 32 || ldo < rows) {
        set_error("prefill gemm: bad rows=%d cols=%d T=%d group=%d bits=%d", rows, cols, T, group, bits);
        return L2Q_ERR_ARG;
    }
    if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(xqp) % 16 ||
        reinterpret_cast<uintptr_t>(rec) % 16 || (size_t)cols * bits / 8 % 16) {
        set_error("prefill gemm: weights, activations and records must be 16-byte aligned (rows of 16n bytes)");
        return L2Q_ERR_ARG;
    }
    // the tile by how many workgroups its grid gives each CU (see PfShape)
    int ncu = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
        ncu = 256;
    const long long wg_wide = (long long)((rows + 63) / 64) * ((T + 63) / 64);
    const long long wg_mid = (long long)((rows + 63) / 64) * ((T + 31) / 32);
    const PfShape shp = wg_wide >= 2 * ncu ? kPfWide : wg_wide >= ncu ? kPfNarrow : wg_mid >= ncu ? kPfMid : kPfSmall;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    if (swiglu) {
        const PfOperand& so = *swiglu;
        if (rope || !so.xqp || !so.rec || reinterpret_cast<uintptr_t>(so.rec) % 16 || (so.bits != 4 && so.bits != 8) ||
            rows % (2 * group) || so.K != rows / 2 || so.T != T) {
            set_error("prefill gemm: bad SwiGLU operand (rows=%d K=%d T=%d)", rows, so.K, so.T);
            return L2Q_ERR_ARG;
        }
        if (bits == 4 && group == 64) pf3_swiglu<4, 64>(wb, ws, rows, cols, xqp, rec, T, so, st);
        if (bits == 4 && group == 32) pf3_swiglu<4, 32>(wb, ws, rows, cols, xqp, rec, T, so, st);
        if (bits == 8 && group == 64) pf3_swiglu<8, 64>(wb, ws, rows, cols, xqp, rec, T, so, st);
        if (bits == 8 && group == 32) pf3_swiglu<8, 32>(wb, ws, rows, cols, xqp, rec, T, so, st);
        return check_launch("prefill_gemm_swiglu");
    }
    if (rope) {
        const PfRope& r = *rope;
        if (!r.rope || !r.kcache || !r.vcache || r.hs <= 0 || r.hs % 2 || r.dim % r.hs || r.kv_dim % r.hs ||
            r.kv_dim > r.dim || rows != r.dim + 2 * r.kv_dim || r.pos0 < 0 || r.row0 < 0 || r.row0 + T > r.max_t ||
            (r.k_il && r.hs % 4)) {
            set_error("prefill gemm: bad RoPE/KV epilogue arguments");
            return L2Q_ERR_ARG;
        }
        pf3_bits<1>(bits, group, shp, wb, ws, rows, cols, xqp, rec, T, out, ldo, r, st);
    } else {
        pf3_bits<0>(bits, group, shp, wb, ws, rows, cols, xqp, rec, T, out, ldo, PfRope{}, st);
    }
    return check_launch("prefill_gemm");
}

int launch_pf_embed(const float* emb, const int* tokens, float* x, int dim, int T, hipStream_t st) {
    hipLaunchKernelGGL(k_pf_embed, dim3((dim + 255) / 256, T), dim3(256), 0, st, emb, tokens, x, dim);
    return check_launch("prefill_embed");
}


int launch_argmax(const float* v, int n, int* out, hipStream_t st) {
    if (n <= 0 || !v || !out || reinterpret_cast<uintptr_t>(v) % 16) {
        set_error("argmax: n=%d (v must be 16-byte aligned)", n);
        return L2Q_ERR_ARG;
    }
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(kArgmaxThreads), 0, st, v, n, out);
    return check_launch("argmax");
}

int launch_unbias(const uint8_t* src, int8_t* dst, size_t n, hipStream_t st) {
    if (n == 0) return L2Q_OK;
    const size_t threads = (n + 15) / 16;
    hipLaunchKernelGGL(k_unbias, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, src, dst, n);
    return check_launch("unbias");
}

// Split counts for a one-off attention call.
static int attention_splits(int pos) {     // split-context path: ~128 positions per workgroup
    int S = (pos + 1 + 127) / 128;
    return S < 1 ? 1 : (S > 512 ? 512 : S);
}

// Per-device scratch for the partials of l2q_attention (grown on demand).
struct AttnScratch {
    float* buf = nullptr;
    size_t floats = 0;
};
static AttnScratch g_attn_scratch[64];

static int attn_scratch(size_t floats, float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) { set_error("attention: device %d out of range", dev); return L2Q_ERR_ARG; }
    AttnScratch& s = g_attn_scratch[dev];
    if (s.floats < floats) {
        if (s.buf) {
            e = hipDeviceSynchronize();
            if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
            (void)hipFree(s.buf);
            s.buf = nullptr;
            s.floats = 0;
        }
        e = hipMalloc(&s.buf, floats * sizeof(float));
        if (e != hipSuccess) { s.buf = nullptr; return hip_fail(e, "hipMalloc(attention scratch)"); }
        s.floats = floats;
    }
    *out = s.buf;
    return L2Q_OK;
}

// The instantiated one-kernel step: the Llama-2-7B shape.
constexpr int kStepD = 4096, kStepH = 11008, kStepHs = 128;

bool step_shape_ok(int d, int h, int hs) { return d == kStepD && h == kStepH && hs == kStepHs; }

size_t step_lds_bytes() { return (size_t)StepShape<kStepD, kStepH, kStepHs>::kTotal * sizeof(float); }

int step_prepare(size_t lds, int* per_cu) {
    const void* fn = reinterpret_cast<const void*>(&k_step<kStepD, kStepH, kStepHs>);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(step)");
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, fn, kStepThreads, lds);
    if (e != hipSuccess) return hip_fail(e, "occupancy(step)");
    return L2Q_OK;
}

#ifdef L2Q_STEP_TRACE
extern "C" int l2q_step_trace_read(void* dst, size_t bytes) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_step_trace), bytes) == hipSuccess ? 0 : -2;
}
#endif

int launch_step_kernel(const StepArgs& a, int grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((k_step<kStepD, kStepH, kStepHs>), dim3(grid), dim3(kStepThreads), lds, st, a);
    return check_launch("step");
}

// Device scratch of l2q_attention_split_noalloc: a file-scope array, one copy
// per GPU, held until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kNoAllocScratchFloats = (size_t)1 << 20;   // 4 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];
static float* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static int noalloc_scratch(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) { set_error("attention: device %d out of range", dev); return L2Q_ERR_ARG; }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return L2Q_OK;
}

}  // namespace l2q

using namespace l2q;

// ---------------------------------------------------------------------------
// C ABI

extern "C" {

const char* l2q_last_error(void) { return g_err; }

int l2q_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int l2q_quantize_act(const float* x, int n, int group, int8_t* xq, float* xs, void* stream) {
    return launch_quantize(x, n, group, xq, xs, (hipStream_t)stream);
}

int l2q_gemv_q8(float* out, const int8_t* xq, const float* xs, const int8_t* w, const float* ws, int rows, int cols,
                int group, int32_t* dots, void* stream) {
    GemvArgs a{};
    a.out = out; a.xq = xq; a.xs = xs; a.w = w; a.ws = ws; a.rows = rows; a.cols = cols; a.dots = dots;
    return launch_gemv(8, group, a, (hipStream_t)stream);
}

int l2q_gemv_q4(float* out, const int8_t* xq, const float* xs, const uint8_t* w, const float* ws, int rows, int cols,
                int group, int32_t* dots, void* stream) {
    GemvArgs a{};
    a.out = out; a.xq = xq; a.xs = xs; a.w = w; a.ws = ws; a.rows = rows; a.cols = cols; a.dots = dots;
    return launch_gemv(4, group, a, (hipStream_t)stream);
}

int l2q_unbias_q8(const uint8_t* src, int8_t* dst, size_t n, void* stream) {
    return launch_unbias(src, dst, n, (hipStream_t)stream);
}

int l2q_rmsnorm_quant(const float* x, const float* resid, float* xout, const float* w, int n, int group, int8_t* xq,
                      float* xs, void* stream) {
    return launch_rmsnorm_quant(x, nullptr, nullptr, resid, xout, w, n, group, xq, xs, (hipStream_t)stream);
}

int l2q_swiglu_quant(const float* hb, const float* hb2, int n, int group, int8_t* xq, float* xs, float* gout,
                     void* stream) {
    return launch_swiglu_quant(hb, hb2, n, group, xq, xs, gout, (hipStream_t)stream);
}

int l2q_rope_kv_append(float* q, const float* k, const float* v, float* kcache, float* vcache, const float* rope,
                       int pos, int n_heads, int n_kv_heads, int head_size, int max_t, void* stream) {
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads) {
        set_error("rope_kv_append: bad heads %d/%d", n_heads, n_kv_heads);
        return L2Q_ERR_ARG;
    }
    return launch_rope_kv_append(q, k, v, kcache, vcache, rope, nullptr, pos, n_heads * head_size,
                                 n_kv_heads * head_size, head_size, max_t, (hipStream_t)stream);
}

// Per-device counters of the split-context attention (zeroed when
// allocated; every launch leaves them zeroed).
struct FlashCounters {
    unsigned* buf = nullptr;
    int n = 0;
};
static FlashCounters g_flash_cnt[64];
static std::mutex g_flash_mu;

static int flash_counters(int n, unsigned** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) { set_error("attention: device %d out of range", dev); return L2Q_ERR_ARG; }
    std::lock_guard<std::mutex> lock(g_flash_mu);
    FlashCounters& c = g_flash_cnt[dev];
    if (c.n < n) {
        if (c.buf) {
            e = hipDeviceSynchronize();
            if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
            (void)hipFree(c.buf);
            c.buf = nullptr;
            c.n = 0;
        }
        e = hipMalloc(&c.buf, (size_t)n * sizeof(unsigned));
        if (e != hipSuccess) { c.buf = nullptr; return hip_fail(e, "hipMalloc(attention counters)"); }
        e = hipMemset(c.buf, 0, (size_t)n * sizeof(unsigned));
        if (e != hipSuccess) return hip_fail(e, "hipMemset(attention counters)");
        c.n = n;
    }
    *out = c.buf;
    return L2Q_OK;
}

int l2q_attention_ex(const float* q, const float* kcache, const float* vcache, float* out, int pos, int n_heads,
                     int n_kv_heads, int head_size, int max_t, int flags, void* stream) {
    const int one = flags & L2Q_ATTN_ONE_KERNEL, two = flags & L2Q_ATTN_TWO_KERNELS;
    const int sc = flags & L2Q_ATTN_SPLIT_CONTEXT;
    if (!attention_shape_ok(n_heads, n_kv_heads, head_size) || pos < 0 || pos >= max_t ||
        (flags & ~(L2Q_ATTN_K_INTERLEAVED | L2Q_ATTN_ONE_KERNEL | L2Q_ATTN_TWO_KERNELS | L2Q_ATTN_SPLIT_CONTEXT)) ||
        (one && two) || (one && !attention_fused_ok(head_size)) || (sc && (one || two)) ||
        (sc && !attention_flash_ok(head_size))) {
        set_error("attention: bad shape or flags heads=%d kv_heads=%d hs=%d pos=%d max_t=%d flags=%d", n_heads,
                  n_kv_heads, head_size, pos, max_t, flags);
        return L2Q_ERR_ARG;
    }
    float* scratch = nullptr;
    int rc;
    if (sc) {
        int dev = 0, ncu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            ncu = 0;
        const int S = attention_flash_splits(n_heads, pos + 1, ncu);
        unsigned* cnt = nullptr;
        if ((rc = attn_scratch(attention_flash_part_floats(n_heads, S, head_size), &scratch))) return rc;
        if ((rc = flash_counters(n_heads, &cnt))) return rc;
        return launch_attention_flash(q, kcache, vcache, out, scratch, cnt, S, nullptr, pos, n_heads, n_kv_heads,
                                      head_size, max_t, flags & L2Q_ATTN_K_INTERLEAVED ? 1 : 0, (hipStream_t)stream);
    }
    if ((rc = attn_scratch((size_t)n_heads * max_t, &scratch))) return rc;
    return launch_attention_exact(q, kcache, vcache, out, scratch, score_splits(pos + 1), nullptr, pos, n_heads,
                                  n_kv_heads, head_size, max_t, (hipStream_t)stream, 1, 0, one ? 1 : two ? 0 : -1,
                                  flags & L2Q_ATTN_K_INTERLEAVED ? 1 : 0);
}

int l2q_attention(const float* q, const float* kcache, const float* vcache, float* out, int pos, int n_heads,
                  int n_kv_heads, int head_size, int max_t, void* stream) {
    return l2q_attention_ex(q, kcache, vcache, out, pos, n_heads, n_kv_heads, head_size, max_t, 0, stream);
}

int l2q_gemm_q(int wbits, float* out, const int8_t* xq, const float* xs, const void* w, const float* ws, int rows,
               int cols, int group, int T, void* stream) {
    if ((wbits != 4 && wbits != 8) || (group != 32 && group != 64) || rows < 1 || T < 1 || cols <= 0 ||
        cols % group || cols % 8 || !out || !xq || !xs || !w || !ws) {
        set_error("gemm: bad arguments bits=%d rows=%d cols=%d group=%d T=%d", wbits, rows, cols, group, T);
        return L2Q_ERR_ARG;
    }
    // scratch: permuted activations (rounded up to 16 bytes), then one
    // record per (group, token)
    const size_t nbt = (size_t)T * (cols / group);
    const size_t xwords = ((size_t)T * cols + 15) / 16 * 4;
    float* scratch = nullptr;
    int rc = attn_scratch(xwords + nbt * sizeof(PfRecord) / 4, &scratch);
    if (rc) return rc;
    int8_t* xqp = reinterpret_cast<int8_t*>(scratch);
    PfRecord* rec = reinterpret_cast<PfRecord*>(scratch + xwords);
    hipStream_t st = (hipStream_t)stream;
    if ((rc = launch_pf_prep(wbits, group, xq, xs, cols, T, xqp, rec, st))) return rc;
    return launch_pf_gemm(wbits, group, w, ws, rows, cols, xqp, rec, T, out, rows, st);
}

int l2q_kv8_append(const float* k, const float* v, int8_t* kcache8, int8_t* vcache8, float* kscale, float* vscale,
                   const float* rope, int pos, int n_kv_heads, int head_size, int max_t, void* stream) {
    return launch_kv8_append(k, v, kcache8, vcache8, kscale, vscale, rope, nullptr, pos, n_kv_heads, head_size, max_t,
                             (hipStream_t)stream);
}

int l2q_attention_kv8_ex(const float* q, const int8_t* kcache8, const int8_t* vcache8, const float* kscale,
                         const float* vscale, float* out, int pos, int n_heads, int n_kv_heads, int head_size,
                         int max_t, int flags, void* stream) {
    if (flags & ~L2Q_ATTN_SPLIT_CONTEXT) {
        set_error("attention kv8: unknown flags %d", flags);
        return L2Q_ERR_ARG;
    }
    if (!flags)
        return l2q_attention_kv8(q, kcache8, vcache8, kscale, vscale, out, pos, n_heads, n_kv_heads, head_size,
                                 max_t, stream);
    if (!kv8_shape_ok(n_heads, n_kv_heads, head_size, max_t) || pos < 0 || pos >= max_t) {
        set_error("attention kv8: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d", n_heads, n_kv_heads,
                  head_size, pos, max_t);
        return L2Q_ERR_ARG;
    }
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        ncu = 0;
    const int S = attention_flash_splits(n_heads, pos + 1, ncu);
    float* scratch = nullptr;
    unsigned* cnt = nullptr;
    int rc;
    if ((rc = attn_scratch(attention_flash_part_floats(n_heads, S, head_size), &scratch))) return rc;
    if ((rc = flash_counters(n_heads, &cnt))) return rc;
    return launch_attention_kv8_split(q, nullptr, nullptr, const_cast<int8_t*>(kcache8), const_cast<int8_t*>(vcache8),
                                      const_cast<float*>(kscale), const_cast<float*>(vscale), out, scratch, cnt, S,
                                      nullptr, pos, n_heads, n_kv_heads, head_size, max_t, (hipStream_t)stream);
}

int l2q_attention_kv8(const float* q, const int8_t* kcache8, const int8_t* vcache8, const float* kscale,
                      const float* vscale, float* out, int pos, int n_heads, int n_kv_heads, int head_size, int max_t,
                      void* stream) {
    if (!kv8_shape_ok(n_heads, n_kv_heads, head_size, max_t) || pos < 0 || pos >= max_t) {
        set_error("attention kv8: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d", n_heads, n_kv_heads,
                  head_size, pos, max_t);
        return L2Q_ERR_ARG;
    }
    // no staging rows: the caches are only read
    return launch_attention_kv8(q, const_cast<int8_t*>(kcache8), const_cast<int8_t*>(vcache8),
                                const_cast<float*>(kscale), const_cast<float*>(vscale), out, nullptr, nullptr, pos,
                                n_heads, n_kv_heads, head_size, max_t, (hipStream_t)stream);
}

int l2q_attention_split(const float* q, const float* kcache, const float* vcache, float* out, int pos, int n_heads,
                        int n_kv_heads, int head_size, int max_t, void* stream) {
    if (!attention_shape_ok(n_heads, n_kv_heads, head_size) || pos < 0 || pos >= max_t) {
        set_error("attention: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d", n_heads, n_kv_heads, head_size,
                  pos, max_t);
        return L2Q_ERR_ARG;
    }
    const int S = attention_splits(pos);
    float* scratch = nullptr;
    int rc = attn_scratch((size_t)n_heads * S * (head_size + 2), &scratch);
    if (rc) return rc;
    return launch_attention_split(q, kcache, vcache, out, scratch, scratch + (size_t)n_heads * S * head_size, S,
                                  nullptr, pos, n_heads, n_kv_heads, head_size, max_t, (hipStream_t)stream);
}

int l2q_attention_split_noalloc(const float* q, const float* kcache, const float* vcache, float* out, int pos,
                                int n_heads, int n_kv_heads, int head_size, int max_t, void* stream) {
    if (!attention_shape_ok(n_heads, n_kv_heads, head_size) || pos < 0 || pos >= max_t) {
        set_error("attention: bad shape heads=%d kv_heads=%d hs=%d pos=%d max_t=%d", n_heads, n_kv_heads, head_size,
                  pos, max_t);
        return L2Q_ERR_ARG;
    }
    const int S = attention_splits(pos);
    const size_t need = (size_t)n_heads * S * (head_size + 2);
    if (need > kNoAllocScratchFloats) {
        set_error("attention_split_noalloc: %d heads x %d splits x (%d + 2) partial floats exceed the %zu-float "
                  "static scratch",
                  n_heads, S, head_size, kNoAllocScratchFloats);
        return L2Q_ERR_ARG;
    }
    float* buf = nullptr;
    int rc = noalloc_scratch(&buf);
    if (rc) return rc;
    return launch_attention_split(q, kcache, vcache, out, buf, buf + (size_t)n_heads * S * head_size, S, nullptr, pos,
                                  n_heads, n_kv_heads, head_size, max_t, (hipStream_t)stream);
}

int l2q_argmax(const float* v, int n, int* out, void* stream) {
    return launch_argmax(v, n, out, (hipStream_t)stream);
}

int l2q_expf(const float* x, float* y, size_t n, void* stream) {
    if (n == 0) return L2Q_OK;
    if (!x || !y) { set_error("expf: null pointer"); return L2Q_ERR_ARG; }
    hipLaunchKernelGGL(k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, y, n);
    return check_launch("expf");
}

void l2q_rope_table(float* table, int max_t, int head_size) {
    for (int pos = 0; pos < max_t; pos++)
        for (int hd = 0; hd < head_size; hd += 2) {
            float freq = 1.0f / powf(10000.0f, hd / (float)head_size);
            float val = pos * freq;
            table[(size_t)pos * head_size + hd] = cosf(val);
            table[(size_t)pos * head_size + hd + 1] = sinf(val);
        }
}

}  // extern "C"
