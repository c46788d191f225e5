/*
 * C ABI of the MI355X (gfx950) native LIF training library, libatlas_train_hip.so.
 *
 * b2_train_hip_v2 has the signature, buffer sizes, metadata and parameter
 * layouts and return codes of the reference's b2_train_cuda_v2
 * (brian2-rust/python/brian2_rust/training_cuda.cu:92-101; caller
 * brian2-rust/src/training/gpu.rs:544-564, metadata gpu.rs:286-341, parameters
 * gpu.rs:454-462).  The library is also exported under the reference symbol
 * b2_train_cuda_v2 so that the reference host (dlopen of B2_TRAIN_CUDA_LIB,
 * gpu.rs:153-172) can load it unchanged.  Supported plans: the dense layered
 * LIF plan (v1) and the projection-graph LIF plan (v2: meta[10] = G edges
 * (input flag, source, target, parameter) at meta[84 + 4e], tied parameter
 * ids; atlas_graph_bptt of training_metal.metal:190-263, meta gpu.rs:319-333);
 * plans with equations, trainable thresholds, phases or noise (meta[11], [14],
 * [15], [79..83] set) return 7 with a message.  Device: B2_TRAIN_HIP_DEVICE
 * (else B2_TRAIN_CUDA_DEVICE), default 0.
 *
 * Return codes (training_cuda.cu:16-95): 0 ok, 1 device, 2 allocation,
 * 3 upload, 4 kernel, 5 readback, 7 invalid plan or host exception; the message
 * is written into (error, capacity).  Device buffers live for one call.
 *
 * Buffers (B batch, T ticks, I inputs, N neurons, E weights, C classes):
 *   meta u64[meta[12]], params f32[2L + 3] = beta[L], theta[L], slope, scale, logit_scale,
 *   x f32[B*T*I], w f32[E], initial f32[B*N], labels u64[B];
 *   out: pre f32[B*T*N] (v2: f32[2*B*T*N], u then the membrane after the tick's edges),
 *   spikes f32[B*T*N], membrane f32[B*N], gradients f32[B*E]
 *   (per sample), initial_grad f32[B*N], logits f32[B*C], losses f32[B].
 */
#ifndef ATLAS_TRAIN_H
#define ATLAS_TRAIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int b2_train_hip_v2(const uint64_t* meta, const float* params, const float* x, const float* w,
                    const float* initial, const uint64_t* labels, float* pre, float* spikes,
                    float* membrane, float* gradients, float* initial_grad, float* logits,
                    float* losses, char* error, size_t capacity);

/* The same entry point under the reference symbol (training_cuda.cu:92). */
int b2_train_cuda_v2(const uint64_t* meta, const float* params, const float* x, const float* w,
                     const float* initial, const uint64_t* labels, float* pre, float* spikes,
                     float* membrane, float* gradients, float* initial_grad, float* logits,
                     float* losses, char* error, size_t capacity);

/* Capability probe required by the reference host for every plan (gpu.rs:84-88). */
uint64_t b2_train_math_v1(void);

/* b2_train_hip_v2 without any device allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate (tight training or serving loops, harnesses that forbid
 * hipMalloc).  It is not capturable into a HIP graph: like b2_train_hip_v2 it copies host
 * buffers synchronously and synchronizes the device.  Every per-call device buffer (staged inputs, outputs before read-back, tapes) is
 * carved out of one static 64 MiB device workspace per GPU (256-byte aligned pieces); a plan
 * that needs more returns 2 with a message.  Same arguments, results and return codes as
 * b2_train_hip_v2.  All calls on one GPU share that GPU's workspace, which keeps the last
 * call's contents: calls that overlap on one GPU (from several host threads) race. */
int b2_train_hip_v2_static(const uint64_t* meta, const float* params, const float* x, const float* w,
                           const float* initial, const uint64_t* labels, float* pre, float* spikes,
                           float* membrane, float* gradients, float* initial_grad, float* logits,
                           float* losses, char* error, size_t capacity);

/*
 * Recurrent spiking-network trainer (the benchmark's configuration 4).  The
 * reference's v2 ABI has no recurrent current-based layer, leaky non-spiking
 * readout or max-over-time loss, so this plan has its own resident interface:
 * weights, Adam moments, the current batch and the tapes stay on the device.
 * Model: h1_t = x_t W_in + s_{t-1} W_rec; s_t = [mem_t > threshold];
 * syn' = alpha syn + h1_t; mem' = (beta mem + syn)(1 - s_t); readout
 * F' = alpha F + s_t W_out, U' = beta U + F; logits = max_t U_t; mean
 * cross-entropy; BPTT with the surrogate 1/(slope |mem - threshold| + 1)^2 and
 * the reset not differentiated; Adam with bias correction.  Weights are
 * row-major (source, target): W_in inputs x hidden, W_rec hidden x hidden,
 * W_out hidden x classes.  batch and hidden must be multiples of 16.
 */
typedef struct {
    uint64_t batch, time, inputs, hidden, classes;
    float alpha, beta, threshold, slope;
    float learning_rate, beta1, beta2, epsilon;
} AtlasRsnnSpec;

typedef struct AtlasRsnn AtlasRsnn;

int atlas_rsnn_create(const AtlasRsnnSpec* spec, const float* w_in, const float* w_rec, const float* w_out,
                      AtlasRsnn** out, char* error, size_t capacity);
void atlas_rsnn_destroy(AtlasRsnn* trainer);
/* Upload a batch: x f32[batch * time * inputs] sample-major, labels u64[batch]. */
int atlas_rsnn_set_batch(AtlasRsnn* trainer, const float* x, const uint64_t* labels, char* error,
                         size_t capacity);
/* Run `repeats` forward (+ backward and Adam when train != 0) passes over the
 * resident batch; losses f32[batch] and logits f32[batch * classes] of the last
 * pass (either may be NULL); device_ms is the HIP-event time of the passes. */
int atlas_rsnn_step(AtlasRsnn* trainer, int train, uint64_t repeats, float* losses, float* logits,
                    double* device_ms, char* error, size_t capacity);
/* One step like atlas_rsnn_step (repeats 1) with HIP events between its phases on the
 * trainer's stream; phase_ms[ATLAS_RSNN_PHASES] receives 0 input GEMM (+ state clear),
 * 1 forward ticks (`time` launches of the recurrent MFMA kernel), 2 readout GEMM, readout and
 * loss, 3 readout adjoint and its GEMM, 4 backward ticks (`time` launches), 5 weight-gradient
 * GEMMs, 6 Adam (3-6 are 0 when train == 0). */
#define ATLAS_RSNN_PHASES 7
int atlas_rsnn_profile(AtlasRsnn* trainer, int train, double* phase_ms, char* error, size_t capacity);
/* Copy a resident buffer: 0-2 weights (in, rec, out), 3-5 their last gradients,
 * 6 spike tape f32[time * batch * hidden], 7 membrane tape (same shape). */
int atlas_rsnn_read(AtlasRsnn* trainer, uint32_t what, float* host, uint64_t count, char* error,
                    size_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_TRAIN_H */
