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
 * LIF plan (meta[10], [11], [14], [15], [80..83] zero); others return 7 with a
 * message.  Device: B2_TRAIN_HIP_DEVICE (else B2_TRAIN_CUDA_DEVICE), default 0.
 *
 * Return codes (training_cuda.cu:16-95): 0 ok, 1 device, 2 allocation,
 * 3 upload, 4 kernel, 5 readback, 7 invalid plan or host exception; the message
 * is written into (error, capacity).  Device buffers live for one call.
 *
 * Buffers (B batch, T ticks, I inputs, N neurons, E weights, C classes):
 *   meta u64[meta[12]], params f32[2L + 3] = beta[L], theta[L], slope, scale, logit_scale,
 *   x f32[B*T*I], w f32[E], initial f32[B*N], labels u64[B];
 *   out: pre f32[B*T*N], spikes f32[B*T*N], membrane f32[B*N], gradients f32[B*E]
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

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_TRAIN_H */
