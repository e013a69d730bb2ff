/*
 * C restatement of the reference's CPU MoE layer — TEST INFRASTRUCTURE ONLY.
 *
 * Follows QwenCPUModel.moeForward (Sources/SwiftletCore/QwenCPUModel.swift:
 * 500-569) op for op, in f32:
 *   router logits = x . W_router^T over the pre-dequantised router (:506;
 *     the dense layer weights are dequantised once per layer load, :129-177);
 *   softmax (:65-71), insertion top-k with ties to the lower id (:508-522);
 *   the chosen experts dequantised on every call (:524-535, through
 *     Checkpoint.dequantized, Checkpoint.swift:168-209: scale*q then + bias);
 *   per pick: gate/up GEMV, silu(g)*u, down GEMV, out += w*d (:549-557);
 *   shared expert and sigmoid gate (:559-566).
 * It is the CPU baseline of bench.py ("port": the reference's Swift +
 * Accelerate path cannot run on Linux) and a cross-check of oracle/moe_ref.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Built with -ffp-contract=off so that every product and sum is rounded
 * separately, as in the Swift source.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    const uint32_t *w;   /* packed codes of expert 0, row-major            */
    const uint16_t *s;   /* fp16 scales of expert 0                        */
    const uint16_t *b;   /* fp16 biases of expert 0                        */
    int32_t rows, in, group, bits;
    int64_t estride_w;   /* words between experts                          */
    int64_t estride_sb;  /* elements between experts                       */
} oq_mat;

/* fp16 bits -> f32 (exact; Checkpoint.swift:235-236). */
static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t u;
    if (ex == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: man * 2^-24 */
            float f = (float)man * 5.9604644775390625e-8f;
            memcpy(&u, &f, 4);
            u |= sign;
        }
    } else if (ex == 31) {
        u = sign | 0x7F800000u | (man << 13);
    } else {
        u = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Checkpoint.dequantized for one expert: out[r*in + i] = s*q + b. */
static void dequantize_rows(const oq_mat *m, int expert, float *out, int threads) {
    const int per = 32 / m->bits;
    const uint32_t mask = (1u << m->bits) - 1u;
    const int wpr = m->in / per;
    const int gpr = m->in / m->group;
    const uint32_t *w = m->w + (int64_t)expert * m->estride_w;
    const uint16_t *s = m->s + (int64_t)expert * m->estride_sb;
    const uint16_t *b = m->b + (int64_t)expert * m->estride_sb;
#pragma omp parallel for num_threads(threads) schedule(static) if (threads > 1)
    for (int r = 0; r < m->rows; ++r) {
        for (int wi = 0; wi < wpr; ++wi) {
            uint32_t word = w[(int64_t)r * wpr + wi];
            for (int j = 0; j < per; ++j) {
                const int col = wi * per + j;
                const int g = col / m->group;
                const float sc = f16_to_f32(s[(int64_t)r * gpr + g]);
                const float bi = f16_to_f32(b[(int64_t)r * gpr + g]);
                const float prod = sc * (float)(word & mask);
                out[(int64_t)r * m->in + col] = prod + bi;
                word >>= m->bits;
            }
        }
    }
}

/* y = W x for row-major W [rows, in] (the reference calls cblas_sgemv,
 * QwenCPUModel.swift:32-45, whose summation order is unspecified; eight
 * interleaved partial sums here). */
static void matvec(const float *W, int rows, int in, const float *x, float *y, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static) if (threads > 1)
    for (int r = 0; r < rows; ++r) {
        const float *wr = W + (int64_t)r * in;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= in; i += 8)
            for (int k = 0; k < 8; ++k) acc[k] += wr[i + k] * x[i + k];
        float t = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
        for (; i < in; ++i) t += wr[i] * x[i];
        y[r] = t;
    }
}

void oracle_dequantize(const oq_mat *m, int expert, float *out) { dequantize_rows(m, expert, out, 1); }

static float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }  /* :61 */
static float silu(float v) { return v * sigmoid(v); }               /* :62 */

/* Returns 0, or -1 on bad arguments.  scratch must hold
 * 2*I*H + H*I + 3*max(I, Is) + 2*H + E floats. */
int oracle_moe_forward(const float *x, int S, int H, int E, int K, int I, int Is, int norm_topk_prob,
                       int has_shared, const float *router, const oq_mat *gate, const oq_mat *up,
                       const oq_mat *down, const float *sh_gate, const float *sh_up, const float *sh_down,
                       const float *seg, float *out, int32_t *ids, float *weights, float *scratch,
                       int threads) {
    if (!x || !router || !gate || !up || !down || !out || !scratch || K <= 0 || K > E || K > 64) return -1;
    const int mx = I > Is ? I : Is;
    float *gW = scratch;
    float *uW = gW + (int64_t)I * H;
    float *dW = uW + (int64_t)I * H;
    float *gbuf = dW + (int64_t)H * I;
    float *ubuf = gbuf + mx;
    float *dbuf = ubuf + mx;
    float *p = dbuf + H;
    (void)Is;

    for (int s = 0; s < S; ++s) {
        const float *xs = x + (int64_t)s * H;
        float *os = out + (int64_t)s * H;
        /* router logits and softmax (:506, :65-71) */
        matvec(router, E, H, xs, p, threads);
        float m = -INFINITY;
        for (int e = 0; e < E; ++e) m = p[e] > m ? p[e] : m;
        float sum = 0.f;
        for (int e = 0; e < E; ++e) {
            p[e] = expf(p[e] - m);
            sum += p[e];
        }
        for (int e = 0; e < E; ++e) p[e] /= sum;
        /* insertion top-k (:510-520): keep picks sorted by p, stable */
        int pe[64];
        float pp[64];
        int n = 0;
        for (int e = 0; e < E; ++e) {
            if (n < K) {
                int j = n++;
                while (j > 0 && pp[j - 1] < p[e]) { pp[j] = pp[j - 1]; pe[j] = pe[j - 1]; --j; }
                pp[j] = p[e];
                pe[j] = e;
            } else if (p[e] > pp[K - 1]) {
                int j = K - 1;
                while (j > 0 && pp[j - 1] < p[e]) { pp[j] = pp[j - 1]; pe[j] = pe[j - 1]; --j; }
                pp[j] = p[e];
                pe[j] = e;
            }
        }
        float score = 0.f;
        for (int k = 0; k < K; ++k) score += pp[k];
        for (int k = 0; k < H; ++k) os[k] = 0.f;
        for (int k = 0; k < K; ++k) {
            const float w = norm_topk_prob ? pp[k] / score : pp[k];   /* :550 */
            if (ids) ids[(int64_t)s * K + k] = pe[k];
            if (weights) weights[(int64_t)s * K + k] = w;
            /* the chosen expert, dequantised on this call (:526-535) */
            dequantize_rows(gate, pe[k], gW, threads);
            dequantize_rows(up, pe[k], uW, threads);
            dequantize_rows(down, pe[k], dW, threads);
            matvec(gW, I, H, xs, gbuf, threads);
            matvec(uW, I, H, xs, ubuf, threads);
            for (int i = 0; i < I; ++i) gbuf[i] = silu(gbuf[i]) * ubuf[i];
            matvec(dW, H, I, gbuf, dbuf, threads);
            for (int i = 0; i < H; ++i) os[i] += w * dbuf[i];
        }
        if (has_shared) {                                          /* :559-566 */
            matvec(sh_gate, Is, H, xs, gbuf, threads);
            matvec(sh_up, Is, H, xs, ubuf, threads);
            for (int i = 0; i < Is; ++i) gbuf[i] = silu(gbuf[i]) * ubuf[i];
            matvec(sh_down, H, Is, gbuf, dbuf, threads);
            float sg = 0.f;
            for (int i = 0; i < H; ++i) sg += seg[i] * xs[i];
            const float scale = sigmoid(sg);
            for (int i = 0; i < H; ++i) os[i] += scale * dbuf[i];
        }
    }
    return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
