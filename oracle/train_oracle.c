/*
 * CPU oracle of the native LIF training kernel (dense layered and projection-graph plans, v2 ABI).
 *
 * TEST INFRASTRUCTURE ONLY: the checker of libatlas_train_hip.so; only tests/
 * and bench.py's CPU-baseline leg may load it.
 *
 * Restates the reference kernel loop by loop for one sample at a time
 * (brian2-rust/python/brian2_rust/training_metal.metal:46-114, the same
 * algorithm as atlas_lif_bptt in training_kernels.cuh): float32 arithmetic in
 * the reference's order, built with -ffp-contract=off.  The readout's
 * exponential and logarithm are the engines' shared implementations rounded to
 * float32 (atlas_math.h), as on the GPU.
 *
 * Pins (tests/test_training.py): the reference's independent NumPy forward and
 * frozen-anchor finite-difference VJP check (test_native_training.py:18-82) with
 * its vectors and tolerances, plus a float64 finite-difference check of the
 * surrogate linearisation at larger sizes.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "atlas_math.h"

/* Projection-graph plans (meta[10] = G edges at meta[84 + 4e]: input flag, source, target,
 * parameter), atlas_graph_bptt of training_metal.metal:190-263 without equations or trainable
 * thresholds: thresholds of every layer first, then every edge in order, then the zero reset;
 * backward, every edge's VJP in order, then every neuron's.  The pre tape has two planes: u and
 * the membrane after the tick's edges. */
static int oracle_train_graph(const uint64_t *m, const float *p, const float *x, const float *w,
                              const float *initial, const uint64_t *labels, float *pre, float *spike,
                              float *membrane, float *grad, float *initial_grad, float *logits, float *losses) {
    const uint64_t B = m[0], T = m[1], L = m[2], I = m[3], N = m[4], E = m[5], C = m[16 + L], G = m[10];
    const uint64_t cells = B * T * N;
    float *carry = calloc(N, sizeof(float)), *ds = calloc(N, sizeof(float)), *previous = calloc(N, sizeof(float));
    if (!carry || !ds || !previous) { free(carry); free(ds); free(previous); return 2; }
    for (uint64_t b = 0; b < B; b++) {
        const uint64_t base = b * N;
        for (uint64_t k = 0; k < N; k++) { membrane[base + k] = initial[base + k]; carry[k] = 0.0f; }
        for (uint64_t e = 0; e < E; e++) grad[b * E + e] = 0.0f;
        for (uint64_t t = 0; t < T; t++) {
            const uint64_t at = (b * T + t) * N;
            for (uint64_t l = 0; l < L; l++)
                for (uint64_t j = 0; j < m[17 + l]; j++) {
                    const uint64_t k = m[40 + l] + j;
                    const float u = p[l] * membrane[base + k];
                    const float s = (float)(u > p[L + l]);
                    pre[at + k] = u;
                    spike[at + k] = s;
                    membrane[base + k] = m[6] ? u : u - p[L + l] * s;
                }
            for (uint64_t e = 0; e < G; e++) {
                const uint64_t *q = m + 84 + 4 * e;
                const float input = q[0] ? x[(b * T + t) * I + q[1]] : spike[at + q[1]];
                membrane[base + q[2]] += w[q[3]] * input;
            }
            for (uint64_t k = 0; k < N; k++) {
                pre[cells + at + k] = membrane[base + k];
                if (m[6]) membrane[base + k] *= 1.0f - spike[at + k];
            }
        }
        const float scale = p[2 * L + 2];
        for (uint64_t j = 0; j < C; j++) {
            float sum = 0.0f;
            for (uint64_t t = 0; t < T; t++) sum += spike[(b * T + t) * N + m[39 + L] + j] * scale / (float)T;
            logits[b * C + j] = sum;
        }
        float maxlog = -INFINITY;
        for (uint64_t j = 0; j < C; j++) maxlog = fmaxf(maxlog, logits[b * C + j]);
        float denom = 0.0f;
        for (uint64_t j = 0; j < C; j++) denom += atlas_expf(logits[b * C + j] - maxlog);
        losses[b] = maxlog + atlas_logf(denom) - logits[b * C + labels[b]];
        if (m[9] & 1)
            for (uint64_t t = T; t-- > 0;) {
                const uint64_t at = (b * T + t) * N;
                for (uint64_t k = 0; k < N; k++) { ds[k] = 0.0f; previous[k] = 0.0f; }
                for (uint64_t j = 0; j < C; j++) {
                    const float d = (atlas_expf(logits[b * C + j] - maxlog) / denom - (float)(j == labels[b])) / (float)B;
                    ds[m[39 + L] + j] = d * scale / (float)T;
                }
                for (uint64_t e = 0; e < G; e++) {
                    const uint64_t *q = m + 84 + 4 * e;
                    const float g = carry[q[2]] * (m[6] ? 1.0f - spike[at + q[2]] : 1.0f);
                    const float input = q[0] ? x[(b * T + t) * I + q[1]] : spike[at + q[1]];
                    grad[b * E + q[3]] += g * input;
                    if (!q[0]) ds[q[1]] += g * w[q[3]];
                }
                for (uint64_t l = 0; l < L; l++)
                    for (uint64_t j = 0; j < m[17 + l]; j++) {
                        const uint64_t k = m[40 + l] + j;
                        const float u = pre[at + k], s = spike[at + k];
                        const float q = 1.0f + p[2 * L] * fabsf(u - p[L + l]);
                        const float phi = p[2 * L + 1] / (q * q);
                        const float derivative = m[6] ? (1.0f - s - (m[7] ? 0.0f : pre[cells + at + k] * phi))
                                                      : (1.0f - (m[7] ? 0.0f : p[L + l] * phi));
                        previous[k] = p[l] * (carry[k] * derivative + ds[k] * phi);
                    }
                for (uint64_t k = 0; k < N; k++) carry[k] = (t > 0 && t % m[8] == 0) ? 0.0f : previous[k];
            }
        for (uint64_t k = 0; k < N; k++) initial_grad[base + k] = carry[k];
    }
    free(carry); free(ds); free(previous);
    return 0;
}

int oracle_train_v2(const uint64_t *m, const float *p, const float *x, const float *w, const float *initial,
                    const uint64_t *labels, float *pre, float *spike, float *membrane, float *grad,
                    float *initial_grad, float *logits, float *losses) {
    if (m[10]) return oracle_train_graph(m, p, x, w, initial, labels, pre, spike, membrane, grad, initial_grad, logits,
                                         losses);
    const uint64_t B = m[0], T = m[1], L = m[2], I = m[3], N = m[4], E = m[5], C = m[16 + L];
    float *carry = calloc(N, sizeof(float)), *ds = calloc(N, sizeof(float)), *previous = calloc(N, sizeof(float));
    if (!carry || !ds || !previous) { free(carry); free(ds); free(previous); return 2; }
    for (uint64_t b = 0; b < B; b++) {
        const uint64_t base = b * N;
        for (uint64_t k = 0; k < N; k++) { membrane[base + k] = initial[base + k]; carry[k] = 0.0f; }
        for (uint64_t e = 0; e < E; e++) grad[b * E + e] = 0.0f;
        for (uint64_t t = 0; t < T; t++) {
            const uint64_t at = (b * T + t) * N;
            for (uint64_t l = 0; l < L; l++)
                for (uint64_t j = 0; j < m[17 + l]; j++) {
                    const uint64_t k = m[40 + l] + j;
                    const float u = p[l] * membrane[base + k];
                    const float s = (float)(u > p[L + l]);
                    pre[at + k] = u;
                    spike[at + k] = s;
                    membrane[base + k] = m[6] ? u : u - p[L + l] * s;
                }
            for (uint64_t l = 0; l < L; l++)
                for (uint64_t j = 0; j < m[17 + l]; j++) {
                    const uint64_t k = m[40 + l] + j;
                    for (uint64_t i = 0; i < m[16 + l]; i++) {
                        const float input = l ? spike[at + m[39 + l] + i] : x[(b * T + t) * I + i];
                        membrane[base + k] += w[m[64 + l] + i * m[17 + l] + j] * input;
                    }
                }
            /* the value before the zero reset, which the backward pass of the reference
             * recomputes by re-accumulating the inputs onto u in the same order */
            if (m[6])
                for (uint64_t k = 0; k < N; k++) membrane[base + k] *= 1.0f - spike[at + k];
        }
        const float scale = p[2 * L + 2];
        for (uint64_t j = 0; j < C; j++) {
            float sum = 0.0f;
            for (uint64_t t = 0; t < T; t++) sum += spike[(b * T + t) * N + m[39 + L] + j] * scale / (float)T;
            logits[b * C + j] = sum;
        }
        float maxlog = -INFINITY;
        for (uint64_t j = 0; j < C; j++) maxlog = fmaxf(maxlog, logits[b * C + j]);
        float denom = 0.0f;
        for (uint64_t j = 0; j < C; j++) denom += atlas_expf(logits[b * C + j] - maxlog);
        losses[b] = maxlog + atlas_logf(denom) - logits[b * C + labels[b]];
        if (m[9] & 1)
            for (uint64_t t = T; t-- > 0;) {
                const uint64_t at = (b * T + t) * N;
                for (uint64_t k = 0; k < N; k++) { ds[k] = 0.0f; previous[k] = 0.0f; }
                for (uint64_t j = 0; j < C; j++) {
                    const float d = (atlas_expf(logits[b * C + j] - maxlog) / denom - (float)(j == labels[b])) / (float)B;
                    ds[m[39 + L] + j] = d * scale / (float)T;
                }
                for (uint64_t l = L; l-- > 0;) {
                    for (uint64_t i = 0; i < m[16 + l]; i++)
                        for (uint64_t j = 0; j < m[17 + l]; j++) {
                            const uint64_t k = m[40 + l] + j, e = m[64 + l] + i * m[17 + l] + j;
                            const float g = carry[k] * (m[6] ? 1.0f - spike[at + k] : 1.0f);
                            const float input = l ? spike[at + m[39 + l] + i] : x[(b * T + t) * I + i];
                            grad[b * E + e] += g * input;
                            if (l) ds[m[39 + l] + i] += g * w[e];
                        }
                    for (uint64_t j = 0; j < m[17 + l]; j++) {
                        const uint64_t k = m[40 + l] + j;
                        const float u = pre[at + k], s = spike[at + k];
                        const float q = 1.0f + p[2 * L] * fabsf(u - p[L + l]);
                        const float phi = p[2 * L + 1] / (q * q);
                        float before_reset = u;
                        if (m[6] && !m[7])
                            for (uint64_t i = 0; i < m[16 + l]; i++) {
                                const float input = l ? spike[at + m[39 + l] + i] : x[(b * T + t) * I + i];
                                before_reset += w[m[64 + l] + i * m[17 + l] + j] * input;
                            }
                        const float derivative = m[6] ? (1.0f - s - (m[7] ? 0.0f : before_reset * phi))
                                                      : (1.0f - (m[7] ? 0.0f : p[L + l] * phi));
                        previous[k] = p[l] * (carry[k] * derivative + ds[k] * phi);
                    }
                }
                for (uint64_t k = 0; k < N; k++) carry[k] = (t > 0 && t % m[8] == 0) ? 0.0f : previous[k];
            }
        for (uint64_t k = 0; k < N; k++) initial_grad[base + k] = carry[k];
    }
    free(carry); free(ds); free(previous);
    return 0;
}
