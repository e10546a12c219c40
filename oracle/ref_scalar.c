/*
 * ORACLE -- test infrastructure only: the CPU baseline that bench.py times beside the GPU.
 * The product never links or calls this file.
 *
 * A restatement of the reference's portable (non-NEON) CPU expert MLP, the code path its
 * library compiles to on a CPU without NEON, built as the reference builds it: -O2 for the
 * host's own instruction set (kandiga/metal/Makefile:5, "-O2 -march=native"; here through
 * function multi-versioning, so the one build runs on any x86-64 host and picks the FMA
 * variant where the CPU has it).  Follows kandiga/metal/kandiga_cpu_expert.m:
 *   - 3-bit dequant GEMV, scalar path :185-210: per 3-byte pack, eight codes, one fp32
 *     accumulator, acc += (q*scale + bias) * x
 *   - 4-bit dequant GEMV, scalar path :276-296 (nibble n of each word)
 *   - expert MLP, SwiGLU :355-401 (silu(g) = g / (1 + expf(-g)))
 *   - K-way fan-out :522-549: one task per selected expert on a persistent worker pool
 *     (the reference's GCD queue; an OpenMP team here)
 * Scales and biases are bf16 (the only dtype the reference stores) or fp16.
 * Unlike oracle/expert_mlp.c (the checker, whose accumulation order is the NEON one and
 * whose build forbids contraction), this file keeps the compiler's default contraction, as
 * the reference build does.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define RS_GROUP 64

typedef struct {
    const void* w;
    const uint16_t* s;
    const uint16_t* b;
    int64_t w_stride; /* bytes between experts */
    int64_t s_stride; /* uint16 elements between experts */
} rs_proj;

/* Same field layout as oracle_layer in expert_mlp.c (the Python binding shares one struct). */
typedef struct {
    int hidden, inter, bits, scale_bf16, act;
    rs_proj gate, up, down;
} rs_layer;

static inline float rs_bf16(uint16_t v) {
    uint32_t x = (uint32_t)v << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float rs_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, x;
    float f;
    if (exp == 0) {
        f = (float)mant * (1.0f / 16777216.0f);
        memcpy(&x, &f, 4);
        x |= sign;
    } else if (exp == 31) {
        x = sign | 0x7F800000u | (mant << 13);
    } else {
        x = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    memcpy(&f, &x, 4);
    return f;
}

#define RS_CLONES __attribute__((target_clones("arch=haswell", "default")))

RS_CLONES
static void rs_matvec3(const uint8_t* restrict w, const uint16_t* restrict s, const uint16_t* restrict b, int bf16,
                       const float* restrict x, float* restrict out, int out_dim, int in_dim) {
    const int bytes_per_row = in_dim * 3 / 8, ng = in_dim / RS_GROUP, ppg = RS_GROUP / 8;
    for (int row = 0; row < out_dim; row++) {
        const uint8_t* wr = w + (size_t)row * bytes_per_row;
        const uint16_t* sr = s + (size_t)row * ng;
        const uint16_t* br = b + (size_t)row * ng;
        float acc = 0.0f;
        for (int g = 0; g < ng; g++) {
            const float scale = bf16 ? rs_bf16(sr[g]) : rs_f16(sr[g]);
            const float bias = bf16 ? rs_bf16(br[g]) : rs_f16(br[g]);
            const uint8_t* wp = wr + g * ppg * 3;
            for (int p = 0; p < ppg; p++) {
                const uint8_t* t = wp + p * 3;
                const float* xp = x + g * RS_GROUP + p * 8;
                const float v0 = (float)(t[0] & 7), v1 = (float)((t[0] >> 3) & 7);
                const float v2 = (float)(((t[0] >> 6) & 3) | ((t[1] & 1) << 2)), v3 = (float)((t[1] >> 1) & 7);
                const float v4 = (float)((t[1] >> 4) & 7), v5 = (float)(((t[1] >> 7) & 1) | ((t[2] & 3) << 1));
                const float v6 = (float)((t[2] >> 2) & 7), v7 = (float)((t[2] >> 5) & 7);
                acc += (v0 * scale + bias) * xp[0];
                acc += (v1 * scale + bias) * xp[1];
                acc += (v2 * scale + bias) * xp[2];
                acc += (v3 * scale + bias) * xp[3];
                acc += (v4 * scale + bias) * xp[4];
                acc += (v5 * scale + bias) * xp[5];
                acc += (v6 * scale + bias) * xp[6];
                acc += (v7 * scale + bias) * xp[7];
            }
        }
        out[row] = acc;
    }
}

RS_CLONES
static void rs_matvec4(const uint32_t* restrict w, const uint16_t* restrict s, const uint16_t* restrict b, int bf16,
                       const float* restrict x, float* restrict out, int out_dim, int in_dim) {
    const int wpr = in_dim / 8, ng = in_dim / RS_GROUP, ppg = RS_GROUP / 8;
    for (int row = 0; row < out_dim; row++) {
        const uint32_t* wr = w + (size_t)row * wpr;
        const uint16_t* sr = s + (size_t)row * ng;
        const uint16_t* br = b + (size_t)row * ng;
        float acc = 0.0f;
        for (int g = 0; g < ng; g++) {
            const float scale = bf16 ? rs_bf16(sr[g]) : rs_f16(sr[g]);
            const float bias = bf16 ? rs_bf16(br[g]) : rs_f16(br[g]);
            for (int p = 0; p < ppg; p++) {
                const uint32_t packed = wr[g * ppg + p];
                const float* xp = x + g * RS_GROUP + p * 8;
                for (int n = 0; n < 8; n++) acc += ((float)((packed >> (n * 4)) & 0xF) * scale + bias) * xp[n];
            }
        }
        out[row] = acc;
    }
}

static void rs_matvec(const rs_layer* L, const rs_proj* P, int e, const float* x, float* out, int out_dim,
                      int in_dim) {
    const uint8_t* w = (const uint8_t*)P->w + (size_t)e * P->w_stride;
    const uint16_t* s = P->s + (size_t)e * P->s_stride;
    const uint16_t* b = P->b + (size_t)e * P->s_stride;
    if (L->bits == 3)
        rs_matvec3(w, s, b, L->scale_bf16, x, out, out_dim, in_dim);
    else
        rs_matvec4((const uint32_t*)w, s, b, L->scale_bf16, x, out, out_dim, in_dim);
}

static void rs_expert(const rs_layer* L, int e, const float* x, float* y, float* scratch) {
    const int H = L->hidden, I = L->inter;
    float *go = scratch, *uo = scratch + I, *act = scratch + 2 * I;
    rs_matvec(L, &L->gate, e, x, go, I, H);
    rs_matvec(L, &L->up, e, x, uo, I, H);
    for (int i = 0; i < I; i++) act[i] = go[i] / (1.0f + expf(-go[i])) * uo[i];
    rs_matvec(L, &L->down, e, act, y, H, I);
}

/*
 * y[t, k, :] = expert idx[t, k] applied to x[t] (fp16 in, fp32 out), token by token; each
 * token's K experts run as K tasks on min(K, nthreads) threads of one persistent team.
 */
int refscalar_switch_mlp(const rs_layer* L, const uint16_t* x16, const int32_t* idx, int T, int K, float* y,
                         int nthreads) {
    const int H = L->hidden, I = L->inter;
    if (T < 0 || K <= 0 || H % RS_GROUP || I % RS_GROUP || (L->bits != 3 && L->bits != 4)) return -1;
    const int nt = nthreads < 1 ? 1 : (nthreads > K ? K : nthreads);
    float* xf = (float*)malloc(sizeof(float) * (size_t)H);
    float* scr = (float*)malloc(sizeof(float) * 3 * (size_t)I * (size_t)K);
    if (!xf || !scr) {
        free(xf);
        free(scr);
        return -1;
    }
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < H; h++) xf[h] = rs_f16(x16[(size_t)t * H + h]);
#pragma omp parallel for num_threads(nt) schedule(static, 1)
        for (int k = 0; k < K; k++)
            rs_expert(L, idx[(size_t)t * K + k], xf, y + ((size_t)t * K + k) * H, scr + (size_t)k * 3 * I);
    }
    free(xf);
    free(scr);
    return 0;
}
