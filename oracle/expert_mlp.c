/*
 * ORACLE -- test infrastructure only.  A CPU restatement of the reference's expert MLP,
 * used by tests/, the smoke check and the CPU-baseline leg of bench.py as the checker.
 * The product never links or calls this file.
 *
 * Follows kandiga/metal/kandiga_cpu_expert.m:
 *   - dequant GEMV, 3-bit  :105-216  (code bit order of the scalar path :194-201)
 *   - dequant GEMV, 4-bit  :221-299
 *   - expert MLP, SwiGLU   :304-401  (silu(g) = g / (1 + expf(-g)), act = silu(g) * u)
 *   - K-way expert fan-out :522-549  (one task per selected expert, then join)
 *   - fp16 / bf16 I/O      :81-99, :662-719
 * and kandiga/metal/kandiga_cpu_expert_lg.m for generic dimensions (:120-268) and the
 * GELU-tanh gate used when the expert intermediate size is 704 (:210-222).
 *
 * Accumulation order is the one the reference runs on its target (the NEON path):
 * four fp32 lanes, lane j accumulating columns k with k % 4 == j in increasing k,
 * each term fused as acc = fma(fma(q, scale, bias), x, acc), and the row result
 * (lane0 + lane2) + (lane1 + lane3) (vadd low/high then vpadd, :181-183).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off).  fp16 conversions are written
 * out bit by bit so the result does not depend on compiler _Float16 support.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_GROUP 64

typedef struct {
    const void* w;      /* packed codes, MLX layout, row-major */
    const uint16_t* s;  /* scales [rows, in/64] */
    const uint16_t* b;  /* biases [rows, in/64] */
    int64_t w_stride;   /* bytes between experts */
    int64_t s_stride;   /* uint16 elements between experts */
} oracle_proj;

typedef struct {
    int hidden;
    int inter;
    int bits;        /* 3 or 4 */
    int scale_bf16;  /* 1: scales/biases are bf16 bit patterns, 0: fp16 */
    int act;         /* 0: SwiGLU, 1: GELU-tanh gate */
    oracle_proj gate, up, down;
} oracle_layer;

/* ---- 16-bit float conversions (kandiga_cpu_expert.m:81-99) -------------------------- */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, x;
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

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu, mant = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13), rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

static inline float bf16_to_f32(uint16_t v) {
    uint32_t x = (uint32_t)v << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float scale_f32(uint16_t v, int bf16) { return bf16 ? bf16_to_f32(v) : oracle_f16_to_f32(v); }

/* Code of column k in a packed row (MLX bit order). */
static inline uint32_t code_at(const uint8_t* row, int k, int bits) {
    if (bits == 4) {
        uint32_t word;
        memcpy(&word, row + 4 * (k >> 3), 4);
        return (word >> (4 * (k & 7))) & 0xFu;
    }
    const uint8_t* t = row + 3 * (k >> 3);
    uint32_t v = (uint32_t)t[0] | ((uint32_t)t[1] << 8) | ((uint32_t)t[2] << 16);
    return (v >> (3 * (k & 7))) & 7u;
}

/* Dequant GEMV over one expert's projection (kandiga_cpu_expert.m:105-299). */
static inline void matvec(const uint8_t* w, const uint16_t* s, const uint16_t* b, int bf16, int bits,
                          const float* x, float* out, int out_dim, int in_dim) {
    const size_t row_bytes = (size_t)in_dim * (size_t)bits / 8;
    const int ng = in_dim / ORACLE_GROUP;
    for (int r = 0; r < out_dim; r++) {
        const uint8_t* wr = w + (size_t)r * row_bytes;
        const uint16_t* sr = s + (size_t)r * ng;
        const uint16_t* br = b + (size_t)r * ng;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int g = 0; g < ng; g++) {
            const float sc = scale_f32(sr[g], bf16), bi = scale_f32(br[g], bf16);
            for (int c = 0; c < ORACLE_GROUP; c++) {
                const int k = g * ORACLE_GROUP + c;
                const float wv = fmaf((float)code_at(wr, k, bits), sc, bi);
                acc[k & 3] = fmaf(wv, x[k], acc[k & 3]);
            }
        }
        out[r] = (acc[0] + acc[2]) + (acc[1] + acc[3]);
    }
}

/* One expert, one token (kandiga_cpu_expert.m:355-401; lg :190-233). */
__attribute__((target_clones("arch=haswell", "default")))
int oracle_expert_forward(const oracle_layer* L, int expert, const float* x, float* out, float* scratch) {
    const int H = L->hidden, I = L->inter;
    float *go = scratch, *uo = scratch + I, *act = scratch + 2 * I;
    const oracle_proj *G = &L->gate, *U = &L->up, *D = &L->down;
    matvec((const uint8_t*)G->w + expert * G->w_stride, G->s + expert * G->s_stride, G->b + expert * G->s_stride,
           L->scale_bf16, L->bits, x, go, I, H);
    matvec((const uint8_t*)U->w + expert * U->w_stride, U->s + expert * U->s_stride, U->b + expert * U->s_stride,
           L->scale_bf16, L->bits, x, uo, I, H);
    if (L->act == 1) {
        for (int i = 0; i < I; i++) {
            const float g = go[i];
            const float t = 0.7978845608f * (g + 0.044715f * g * g * g);
            act[i] = 0.5f * g * (1 + tanhf(t)) * uo[i];
        }
    } else {
        for (int i = 0; i < I; i++) {
            const float silu = go[i] / (1.0f + expf(-go[i]));
            act[i] = silu * uo[i];
        }
    }
    matvec((const uint8_t*)D->w + expert * D->w_stride, D->s + expert * D->s_stride, D->b + expert * D->s_stride,
           L->scale_bf16, L->bits, act, out, H, I);
    return 0;
}

/* ---- K-way fan-out per token (kandiga_cpu_expert.m:522-549) --------------------------- */
typedef struct {
    const oracle_layer* L;
    const float* x;
    const int32_t* idx;
    int K, tid, nthreads;
    float* y;       /* [K, H] */
    float* scratch; /* 3*I */
    int err;
} fan_task;

static void* fan_worker(void* arg) {
    fan_task* t = (fan_task*)arg;
    for (int k = t->tid; k < t->K; k += t->nthreads)
        if (oracle_expert_forward(t->L, t->idx[k], t->x, t->y + (size_t)k * t->L->hidden, t->scratch)) t->err = 1;
    return NULL;
}

/* One token row of x as fp32: fp16 bits widened (kandiga_cpu_expert.m:670-674), or fp32 as given
 * (bakan_cpu_expert_mlp, :471-552; the bf16 entry widens bf16 to fp32 and calls it, :690-719). */
static void token_row(const uint16_t* x_f16, const float* x_f32, int t, int H, float* xf) {
    for (int h = 0; h < H; h++)
        xf[h] = x_f16 ? oracle_f16_to_f32(x_f16[(size_t)t * H + h]) : x_f32[(size_t)t * H + h];
}

static int switch_mlp_rows(const oracle_layer* L, const uint16_t* x_f16, const float* x_f32, const int32_t* idx,
                           int T, int K, float* y, int nthreads) {
    const int H = L->hidden, I = L->inter;
    if (T < 0 || K <= 0 || H % ORACLE_GROUP || I % ORACLE_GROUP || (L->bits != 3 && L->bits != 4)) return -1;
    int nt = nthreads < 1 ? 1 : (nthreads > K ? K : nthreads);
    float* xf = (float*)malloc(sizeof(float) * (size_t)H);
    float* scr = (float*)malloc(sizeof(float) * 3 * (size_t)I * (size_t)nt);
    if (!xf || !scr) {
        free(xf);
        free(scr);
        return -1;
    }
    int err = 0;
    for (int t = 0; t < T && !err; t++) {
        token_row(x_f16, x_f32, t, H, xf);
        fan_task tasks[64];
        pthread_t th[64];
        if (nt > 64) nt = 64;
        for (int i = 0; i < nt; i++) {
            tasks[i] = (fan_task){L, xf, idx + (size_t)t * K, K, i, nt, y + (size_t)t * K * H, scr + (size_t)i * 3 * I, 0};
        }
        if (nt == 1) {
            fan_worker(&tasks[0]);
        } else {
            for (int i = 0; i < nt; i++) pthread_create(&th[i], NULL, fan_worker, &tasks[i]);
            for (int i = 0; i < nt; i++) pthread_join(th[i], NULL);
        }
        for (int i = 0; i < nt; i++) err |= tasks[i].err;
    }
    free(xf);
    free(scr);
    return err ? -1 : 0;
}

/*
 * switch_mlp contract (kandiga/engine.py:670-739): y[t, k, :] = expert idx[t, k] applied to x[t].
 * x is fp16 [T, H] (converted to fp32 as kandiga_cpu_expert.m:670-674), y is fp32 [T, K, H]
 * (the value bakan_cpu_expert_mlp returns before its fp16 rounding).
 * nthreads <= 1 runs single-threaded; otherwise each token fans its K experts over
 * min(K, nthreads) threads and joins before the next token, as the reference does.
 */
int oracle_switch_mlp(const oracle_layer* L, const uint16_t* x_f16, const int32_t* idx, int T, int K, float* y,
                      int nthreads) {
    return x_f16 ? switch_mlp_rows(L, x_f16, NULL, idx, T, K, y, nthreads) : -1;
}

/* The same with fp32 activations [T, H] taken as they are (bakan_cpu_expert_mlp). */
int oracle_switch_mlp_f32(const oracle_layer* L, const float* x_f32, const int32_t* idx, int T, int K, float* y,
                          int nthreads) {
    return x_f32 ? switch_mlp_rows(L, NULL, x_f32, idx, T, K, y, nthreads) : -1;
}

/* fp32 -> fp16 rounding of a buffer (kandiga_cpu_expert.m:681-685). */
void oracle_round_f16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = oracle_f32_to_f16(in[i]);
}
