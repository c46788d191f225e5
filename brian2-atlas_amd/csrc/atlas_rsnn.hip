// Recurrent spiking-network trainer (configuration 4 of the benchmark plan):
// 700 Poisson inputs -> 256 recurrent current-based LIF units -> 20 leaky
// non-spiking readout units, max-over-time cross-entropy, full BPTT with a
// fast-sigmoid surrogate, Adam.  Part of libatlas_train_hip.so.
//
// Model (the widely used SpyTorch discretisation; every step reads the states
// entering the tick):
//   h1_t  = x_t W_in + s_{t-1} W_rec                  (s_{-1} = 0)
//   s_t   = H(mem_t - theta)                           surrogate 1/(slope |mem_t - theta| + 1)^2
//   syn_{t+1} = alpha syn_t + h1_t
//   mem_{t+1} = (beta mem_t + syn_t)(1 - s_t)          (reset not differentiated)
//   readout: F_{t+1} = alpha F_t + s_t W_out, U_{t+1} = beta U_t + F_t,
//            logits = max over U_0 .. U_T, loss = mean cross-entropy.
//
// Work split on the MI355X:
//   * the GEMMs that span every tick at once (x W_in, S W_out, the weight
//     gradients X^T G, S^T G and the readout adjoint) are library GEMMs
//     (rocBLAS; bf16 MFMA with split-precision operands where one side is 0/1,
//     else fp32), with rows ordered (tick, sample);
//   * the tick-sequential recurrence s_{t-1} W_rec (and g_{t+1} W_rec^T on the
//     way back) runs in one persistent launch per pass, fused with the LIF
//     update or its adjoint: at H = 256 one sample per workgroup with fp32 FMAs
//     (a GEMV per tick), otherwise four samples per workgroup on fp32 MFMA;
//     beyond H = 256, one launch of tiled 16x16 MFMA kernels per tick;
//   * the readout recurrence, loss and Adam are element-wise kernels.
// Everything stays resident between steps: weights, Adam moments, the current
// batch and the tapes.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <new>

#include "device/atlas_math.h"
#include "../../include/atlas_train.h"

namespace {

typedef uint64_t u64;
typedef int64_t i64;
typedef float float4_t __attribute__((ext_vector_type(4)));

typedef uint16_t bf16_t;

// bfloat16 (round to nearest even) and back; every value here is finite.
__device__ __forceinline__ bf16_t to_bf16(float f) {
    const uint32_t bits = __float_as_uint(f);
    return (bf16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float from_bf16(bf16_t b) { return __uint_as_float((uint32_t)b << 16); }

// f = hi + mid + lo with three bfloat16 pieces; the residuals f - hi and (f - hi) - mid are
// exact in float32 and each piece carries 8 more significant bits, so the split is exact to
// about 2^-25 relative.  A product of a piece with a 0/1 value is exact in a float32 sum, so a
// bf16 MFMA GEMM over the three pieces (float32 accumulation) is as accurate as a float32 GEMM
// whenever the other operand holds only exactly representable values (spikes, binary inputs).
__device__ __forceinline__ void split3(float f, bf16_t& hi, bf16_t& mid, bf16_t& lo) {
    hi = to_bf16(f);
    const float r1 = f - from_bf16(hi);
    mid = to_bf16(r1);
    lo = to_bf16(r1 - from_bf16(mid));
}

int fail(char* err, size_t cap, int code, const char* fmt, ...) {
    if (err && cap) {
        va_list args;
        va_start(args, fmt);
        vsnprintf(err, cap, fmt, args);
        va_end(args);
    }
    return code;
}

inline unsigned blocks(u64 items, unsigned width = 256) { return (unsigned)((items + width - 1) / width); }

// ------------------------------------------------------------ recurrent tick
// One wavefront computes the 16x16 tile (rows b0.., cols h0..) of A(BxK) * W(KxH)
// over K = hidden, with fp32 MFMA.  Lane l supplies A[b0 + l%16][k0 + l/16] and
// W[k0 + l/16][h0 + l%16] per 4-wide K step and receives rows 4(l/16)+j, column l%16.
template <bool TRANSPOSED>
__device__ __forceinline__ float4_t tile_product(const float* __restrict__ a, const float* __restrict__ w, u64 hidden,
                                                 u64 b0, u64 h0, unsigned lane) {
    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* arow = a + (b0 + lane % 16) * hidden + lane / 16;
    for (u64 k0 = 0; k0 < hidden; k0 += 4) {
        const float x = arow[k0];
        // TRANSPOSED: W^T, i.e. element (k, c) read from W[c][k]
        const float y = TRANSPOSED ? w[(h0 + lane % 16) * hidden + k0 + lane / 16]
                                   : w[(k0 + lane / 16) * hidden + h0 + lane % 16];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc, 0, 0, 0);
    }
    return acc;
}

// Forward tick t: spikes from the entering membrane, then the state update with
// h1 = Hin_t + s_{t-1} W_rec.  Tapes: membrane entering the tick and the spikes.
__global__ void __launch_bounds__(256) forward_tick(u64 t, u64 B, u64 H, float alpha, float beta, float theta,
                                                    const float* __restrict__ w_rec, const float* __restrict__ hin,
                                                    float* __restrict__ syn, float* __restrict__ mem,
                                                    float* __restrict__ mem_tape, float* __restrict__ spikes) {
    const unsigned lane = threadIdx.x % 64;
    const u64 tile = (u64)blockIdx.x * 4 + threadIdx.x / 64;
    const u64 tiles_h = H / 16;
    if (tile >= (B / 16) * tiles_h) return;
    const u64 b0 = (tile / tiles_h) * 16, h0 = (tile % tiles_h) * 16;
    float4_t rec = {0.0f, 0.0f, 0.0f, 0.0f};
    if (t > 0) rec = tile_product<false>(spikes + (t - 1) * B * H, w_rec, H, b0, h0, lane);
    for (int j = 0; j < 4; ++j) {
        const u64 b = b0 + 4 * (lane / 16) + j, h = h0 + lane % 16;
        const u64 at = b * H + h, tb = t * B * H + at;
        const float m = mem[at], sy = syn[at];
        const float s = m > theta ? 1.0f : 0.0f;
        mem_tape[tb] = m;
        spikes[tb] = s;
        const float h1 = hin[tb] + rec[j];
        syn[at] = alpha * sy + h1;
        mem[at] = (beta * m + sy) * (1.0f - s);
    }
}

// Backward tick t: gs_t = gs_readout_t + g1_{t+1} W_rec^T; the adjoints of
// (mem_t, syn_t) from those of (mem_{t+1}, syn_{t+1}); g1_t = adjoint of syn_{t+1}.
__global__ void __launch_bounds__(256) backward_tick(u64 t, u64 T, u64 B, u64 H, float alpha, float beta,
                                                     float theta, float slope, const float* __restrict__ w_rec,
                                                     const float* __restrict__ gs_read, const float* __restrict__ mem_tape,
                                                     const float* __restrict__ spikes, float* __restrict__ gmem,
                                                     float* __restrict__ gsyn, float* __restrict__ g1) {
    const unsigned lane = threadIdx.x % 64;
    const u64 tile = (u64)blockIdx.x * 4 + threadIdx.x / 64;
    const u64 tiles_h = H / 16;
    if (tile >= (B / 16) * tiles_h) return;
    const u64 b0 = (tile / tiles_h) * 16, h0 = (tile % tiles_h) * 16;
    float4_t rec = {0.0f, 0.0f, 0.0f, 0.0f};
    if (t + 1 < T) rec = tile_product<true>(g1 + (t + 1) * B * H, w_rec, H, b0, h0, lane);
    for (int j = 0; j < 4; ++j) {
        const u64 b = b0 + 4 * (lane / 16) + j, h = h0 + lane % 16;
        const u64 at = b * H + h, tb = t * B * H + at;
        const float gm_next = gmem[at], gs_next = gsyn[at];
        g1[tb] = gs_next;
        const float s = spikes[tb], m = mem_tape[tb];
        const float q = slope * fabsf(m - theta) + 1.0f;
        const float sigma = 1.0f / (q * q);
        const float gs = gs_read[tb] + rec[j];
        gmem[at] = beta * (1.0f - s) * gm_next + gs * sigma;
        gsyn[at] = (1.0f - s) * gm_next + alpha * gs_next;
    }
}

// ------------------------------------------------- persistent recurrent pass
// The recurrence couples the hidden units of one sample only, so a workgroup can own four
// samples for every tick of a pass with nothing but workgroup barriers between ticks.  Wave w
// owns columns [64w, 64w + 64): lane l holds column h = 64w + l of all four samples (state in
// registers) and the matching slab of W_rec, the B operand of v_mfma_f32_4x4x1f32 (16 blocks of
// 4x4; lane 4b+j gives A_b[j] and B_b[j] and receives D_b[i][j] in acc[i]).  The A operand is
// broadcast (CBSZ = 4: every block takes block ABID's A), so lane 4b+i can hold x_i[16r + b]
// in register r: the instruction with ABID = b then adds x_i[k] W[k][64w + l], k = 16r + b, for
// the four samples i, and a tick is KMAX instructions per wave fed by KMAX / 16 A registers.
// The four samples' vectors of the tick are exchanged through a double-buffered LDS array laid
// out for that: row 4b + i holds x_i[16r + b] at column r (rows padded to a 16-byte multiple
// plus 16 bytes, so that the row-per-lane float4 reads do not conflict), one barrier per tick.
// The slab's first KREG rows live in registers, the remaining KMAX - KREG rows in LDS as float4
// groups of four rows per column (conflict-free 16-byte reads), which leaves registers free for
// the next tick's prefetch.  Columns and rows >= H hold zero weights and zero exchanged values,
// so the product runs over all KMAX rows unbranched.
template <int KMAX>
struct Exchange {
    static constexpr int R = KMAX / 16;   // A registers per lane
    static constexpr int ROW = R + 4;     // floats per padded row
    static constexpr int SIZE = 64 * ROW;

    // column h of sample i
    __device__ static __forceinline__ void put(float* x, u64 h, int i, float v) {
        x[((h % 16) * 4 + i) * ROW + h / 16] = v;
    }
};

template <int KMAX, int KREG>
struct Slab {
    static constexpr int KLDS = KMAX - KREG;
    float w[KREG];
    float4_t* tail;  // LDS: KLDS / 4 groups x KMAX columns

    // FORWARD: B operand W[k][h]; otherwise W^T, i.e. W[h][k]
    template <bool FORWARD>
    __device__ __forceinline__ void load(const float* __restrict__ w_rec, u64 H, u64 h) {
        const bool live = h < H;
#pragma unroll
        for (int k = 0; k < KREG; ++k)
            w[k] = (live && (u64)k < H) ? (FORWARD ? w_rec[(u64)k * H + h] : w_rec[h * H + k]) : 0.0f;
#pragma unroll
        for (int g = 0; g < KLDS / 4; ++g) {
            float4_t v;
            for (int j = 0; j < 4; ++j) {
                const u64 k = (u64)(KREG + 4 * g + j);
                v[j] = (live && k < H) ? (FORWARD ? w_rec[k * H + h] : w_rec[h * H + k]) : 0.0f;
            }
            tail[g * KMAX + h] = v;
        }
    }

    __device__ __forceinline__ float4_t product(const float* __restrict__ x, unsigned lane, u64 h) const {
        typedef Exchange<KMAX> X;
        float a[X::R];
        const float4_t* row = reinterpret_cast<const float4_t*>(x + lane * X::ROW);
#pragma unroll
        for (int q = 0; q < X::R / 4; ++q) {
            const float4_t v = row[q];
            a[4 * q] = v[0];
            a[4 * q + 1] = v[1];
            a[4 * q + 2] = v[2];
            a[4 * q + 3] = v[3];
        }
        float4_t acc[4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f},
                           {0.0f, 0.0f, 0.0f, 0.0f}};
        chain<0>(a, h, acc);
        return (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }

    // rows K .. K + 3 (K + j = 16 r + id: A register r, broadcast block id), then the rest
    template <int K>
    __device__ __forceinline__ void chain(const float* a, u64 h, float4_t* acc) const {
        if constexpr (K < KMAX) {
            float4_t b;
            if constexpr (K < KREG) {
                b[0] = w[K];
                b[1] = w[K + 1];
                b[2] = w[K + 2];
                b[3] = w[K + 3];
            } else {
                b = tail[((K - KREG) / 4) * KMAX + h];
            }
            // row K + j accumulates into acc[j]: consecutive MFMAs are independent, so none waits for
            // the one before it
            constexpr int r = K / 16, id = K % 16;
            acc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[r], b[0], acc[0], 4, id, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[r], b[1], acc[1], 4, id + 1, 0);
            acc[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[r], b[2], acc[2], 4, id + 2, 0);
            acc[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[r], b[3], acc[3], 4, id + 3, 0);
            chain<K + 4>(a, h, acc);
        }
    }
};

// Workgroup barrier ordering LDS only: the tick's global stores and prefetches stay in flight
// (a full __syncthreads() would wait for every outstanding global access each tick).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Forward pass over every tick.  Tick t: P_t = s_t W_rec (used by tick t + 1) and the update
// with h1_t = Hin_t + P_{t-1}; then s_{t+1} from the new membrane, published to LDS and taped
// (tick 0's before the loop).  The update and the next tick's threshold, exchange and tapes do
// not depend on P_t, so they share one block with its MFMA chain (with every work-item live,
// FULL, the block has no branch) and the compiler schedules them together.  Grid: batch / 4
// workgroups of KMAX work-items, H <= KMAX.
template <int KMAX, int KREG, bool FULL>
__global__ void __launch_bounds__(KMAX) forward_pass(u64 T, u64 B, u64 H, float alpha, float beta, float theta,
                                                     const float* __restrict__ w_rec, const float* __restrict__ hin,
                                                     float* __restrict__ mem_tape, float* __restrict__ spikes,
                                                     bf16_t* __restrict__ spikes16) {
    __shared__ __attribute__((aligned(16))) float xs[2][Exchange<KMAX>::SIZE];
    __shared__ float4_t tail[(KMAX - KREG) / 4 * KMAX + 1];
    const unsigned lane = threadIdx.x % 64;
    const u64 h = threadIdx.x, b0 = (u64)blockIdx.x * 4;
    const bool live = FULL || h < H;
    Slab<KMAX, KREG> slab;
    slab.tail = tail;
    slab.template load<true>(w_rec, H, h);
    float syn[4] = {0.0f, 0.0f, 0.0f, 0.0f}, mem[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float s[4], in[4], next[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float4_t rec = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 4; ++i) in[i] = live ? hin[(b0 + i) * H + h] : 0.0f;
    // s_t from the membrane entering tick t, published and taped; tick t + 1's input prefetched
    // (the index is clamped inside the run; the value is unused after the last tick)
    auto emit = [&](u64 t) {
        float* x = xs[t & 1];
        const u64 tn = t + 1 < T ? t + 1 : t;
        for (int i = 0; i < 4; ++i) {
            s[i] = mem[i] > theta ? 1.0f : 0.0f;
            Exchange<KMAX>::put(x, h, i, s[i]);
            if (live) {
                const u64 at = (t * B + b0 + i) * H + h;
                mem_tape[at] = mem[i];
                spikes[at] = s[i];
                spikes16[at] = s[i] != 0.0f ? (bf16_t)0x3F80 : (bf16_t)0;
                next[i] = hin[(tn * B + b0 + i) * H + h];
            }
        }
    };
    auto update = [&]() {
        for (int i = 0; i < 4; ++i) {
            const float h1 = in[i] + rec[i];
            const float sy = syn[i];
            syn[i] = alpha * sy + h1;
            mem[i] = (beta * mem[i] + sy) * (1.0f - s[i]);
            in[i] = next[i];
        }
    };
    emit(0);
    for (u64 t = 0; t < T; ++t) {
        lds_barrier();
        float4_t product = {0.0f, 0.0f, 0.0f, 0.0f};
        if (t + 1 < T) {
            product = slab.product(xs[t & 1], lane, h);
            update();
            emit(t + 1);
        } else {
            update();
        }
        rec = product;
    }
}

// Backward pass over every tick, descending.  Tick t: Q_t = g1_t W_rec^T (used by tick t - 1),
// then the adjoints of (mem_t, syn_t) with gs_t = gs_read_t + Q_{t+1}; then g1_{t-1} (the new
// adjoint of syn) written and published, and tick t - 2's tape values prefetched.  As in the
// forward pass, everything but Q_t shares one block with its MFMA chain.  Lane l holds row h of
// W_rec (the B operand of W_rec^T).
template <int KMAX, int KREG, bool FULL>
__global__ void __launch_bounds__(KMAX) backward_pass(u64 T, u64 B, u64 H, float alpha, float beta, float theta,
                                                      float slope, const float* __restrict__ w_rec,
                                                      const float* __restrict__ gs_read,
                                                      const float* __restrict__ mem_tape,
                                                      const float* __restrict__ spikes, float* __restrict__ g1,
                                                      bf16_t* __restrict__ g3) {
    __shared__ __attribute__((aligned(16))) float xs[2][Exchange<KMAX>::SIZE];
    __shared__ float4_t tail[(KMAX - KREG) / 4 * KMAX + 1];
    const unsigned lane = threadIdx.x % 64;
    const u64 h = threadIdx.x, b0 = (u64)blockIdx.x * 4;
    const bool live = FULL || h < H;
    Slab<KMAX, KREG> slab;
    slab.tail = tail;
    slab.template load<false>(w_rec, H, h);
    float gmem[4] = {0.0f, 0.0f, 0.0f, 0.0f}, gsyn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float4_t rec = {0.0f, 0.0f, 0.0f, 0.0f};
    float gr[4] = {0.0f, 0.0f, 0.0f, 0.0f}, sp[4] = {0.0f, 0.0f, 0.0f, 0.0f}, mt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float ngr[4] = {0.0f, 0.0f, 0.0f, 0.0f}, nsp[4] = {0.0f, 0.0f, 0.0f, 0.0f}, nmt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live)
        for (int i = 0; i < 4; ++i) {
            const u64 at = ((T - 1) * B + b0 + i) * H + h;
            gr[i] = gs_read[at];
            sp[i] = spikes[at];
            mt[i] = mem_tape[at];
        }
    // g1_t (the adjoint of syn_{t+1}) published and written; tick t - 1's tape values prefetched
    // (clamped inside the run; unused before tick 0)
    auto emit = [&](u64 t) {
        float* x = xs[t & 1];
        const u64 tp = t > 0 ? t - 1 : t;
        for (int i = 0; i < 4; ++i) {
            Exchange<KMAX>::put(x, h, i, gsyn[i]);
            if (live) {
                const u64 at = (t * B + b0 + i) * H + h;
                g1[at] = gsyn[i];
                bf16_t* piece = g3 + (t * B + b0 + i) * 3 * H + h;
                split3(gsyn[i], piece[0], piece[H], piece[2 * H]);
                const u64 prev = (tp * B + b0 + i) * H + h;
                ngr[i] = gs_read[prev];
                nsp[i] = spikes[prev];
                nmt[i] = mem_tape[prev];
            }
        }
    };
    auto update = [&]() {
        for (int i = 0; i < 4; ++i) {
            const float q = slope * fabsf(mt[i] - theta) + 1.0f;
            const float sigma = 1.0f / (q * q);
            const float gs = gr[i] + rec[i];
            const float gm_next = gmem[i], gs_next = gsyn[i];
            gmem[i] = beta * (1.0f - sp[i]) * gm_next + gs * sigma;
            gsyn[i] = (1.0f - sp[i]) * gm_next + alpha * gs_next;
            gr[i] = ngr[i];
            sp[i] = nsp[i];
            mt[i] = nmt[i];
        }
    };
    emit(T - 1);
    for (u64 t = T; t-- > 0;) {
        lds_barrier();
        float4_t product = {0.0f, 0.0f, 0.0f, 0.0f};
        if (t > 0) {
            product = slab.product(xs[t & 1], lane, h);
            update();
            emit(t - 1);
        } else {
            update();
        }
        rec = product;
    }
}

// ------------------------------------------------ one sample per workgroup (H = 256)
// The recurrence couples the hidden units of one sample only, and a batch of 256 samples gives
// every CU of the MI355X one.  A 1024-wide workgroup runs all ticks of one sample: column h of
// the product is the dot product of the tick's 256-vector with column h of W_rec (row h of W_rec
// on the way back), split over a quad of lanes by quarters of the rows, each lane holding its 64
// weights in registers and reading its quarter of the vector from LDS (float4 broadcasts; the
// quarters start 68 floats apart, so the quad's four reads hit disjoint banks).  Four
// independent accumulators per lane, then two DPP adds give every lane of the quad the column's
// product; the quad updates the column's state redundantly (identical bits) and its first lane
// writes the tapes and the next tick's vector.  One workgroup barrier per tick.  A GEMV has one
// row, so plain FMAs: an MFMA would leave three of its four (or more) rows empty.
constexpr int VEC_H = 256;
constexpr int VEC_PAD = 4;   // floats between the quarters of the exchanged vector

__device__ __forceinline__ int vec_at(int k) { return k + VEC_PAD * (k / 64); }

// Sum over the quad (lanes 4i .. 4i + 3): every lane ends with ((p0 + p1) + (p2 + p3)) up to the
// order of commutative additions, so with the same bits.
__device__ __forceinline__ float quad_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));   // [1,0,3,2]
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));   // [2,3,0,1]
    return v;
}

// The lane's quarter (rows 64 q .. 64 q + 63) of the product of the exchanged vector x with its
// 64 weights.
__device__ __forceinline__ float quarter_dot(const float* __restrict__ x, const float* w, unsigned q) {
    const float4_t* v = reinterpret_cast<const float4_t*>(x + vec_at(64 * (int)q));
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 16; ++g) {
        const float4_t a = v[g];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(a[j], w[4 * g + j], acc[j]);
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

__global__ void __launch_bounds__(1024) forward_vec(u64 T, u64 B, float alpha, float beta, float theta,
                                                    const float* __restrict__ w_rec, const float* __restrict__ hin,
                                                    float* __restrict__ mem_tape, float* __restrict__ spikes,
                                                    bf16_t* __restrict__ spikes16) {
    constexpr u64 H = VEC_H;
    __shared__ __attribute__((aligned(16))) float xs[2][H + 4 * VEC_PAD];
    const unsigned lane = threadIdx.x % 64, q = lane & 3u;
    const u64 h = (threadIdx.x / 64) * 16 + lane / 4, b = blockIdx.x;
    const bool first = q == 0;
    float w[64];
#pragma unroll
    for (int k = 0; k < 64; ++k) w[k] = w_rec[(64 * q + k) * H + h];
    float syn = 0.0f, mem = 0.0f, s = 0.0f, rec = 0.0f, next = 0.0f;
    float in = hin[b * H + h];
    auto emit = [&](u64 t) {
        const u64 tn = t + 1 < T ? t + 1 : t;
        s = mem > theta ? 1.0f : 0.0f;
        const uint32_t at = (uint32_t)((t * B + b) * H + h);
        if (first) {
            xs[t & 1][vec_at((int)h)] = s;
            mem_tape[at] = mem;
            spikes[at] = s;
            spikes16[at] = s != 0.0f ? (bf16_t)0x3F80 : (bf16_t)0;
        }
        next = hin[(uint32_t)((tn * B + b) * H + h)];
    };
    auto update = [&]() {
        const float h1 = in + rec;
        const float sy = syn;
        syn = alpha * sy + h1;
        mem = (beta * mem + sy) * (1.0f - s);
        in = next;
    };
    emit(0);
    for (u64 t = 0; t < T; ++t) {
        lds_barrier();
        float p = 0.0f;
        if (t + 1 < T) {
            p = quad_sum(quarter_dot(xs[t & 1], w, q));
            update();
            emit(t + 1);
        } else {
            update();
        }
        rec = p;
    }
}

__global__ void __launch_bounds__(1024) backward_vec(u64 T, u64 B, float alpha, float beta, float theta, float slope,
                                                     const float* __restrict__ w_rec,
                                                     const float* __restrict__ gs_read,
                                                     const float* __restrict__ mem_tape,
                                                     const float* __restrict__ spikes, float* __restrict__ g1,
                                                     bf16_t* __restrict__ g3) {
    constexpr u64 H = VEC_H;
    __shared__ __attribute__((aligned(16))) float xs[2][H + 4 * VEC_PAD];
    const unsigned lane = threadIdx.x % 64, q = lane & 3u;
    const u64 h = (threadIdx.x / 64) * 16 + lane / 4, b = blockIdx.x;
    const bool first = q == 0;
    float w[64];
#pragma unroll
    for (int k = 0; k < 64; ++k) w[k] = w_rec[h * H + 64 * q + k];   // row h of W_rec: column h of W_rec^T
    float gmem = 0.0f, gsyn = 0.0f, rec = 0.0f, ngr = 0.0f, nsp = 0.0f, nmt = 0.0f;
    const u64 last = ((T - 1) * B + b) * H + h;
    float gr = gs_read[last], sp = spikes[last], mt = mem_tape[last];
    auto emit = [&](u64 t) {
        const u64 tp = t > 0 ? t - 1 : t;
        if (first) {
            xs[t & 1][vec_at((int)h)] = gsyn;
            const uint32_t at = (uint32_t)((t * B + b) * H + h);
            g1[at] = gsyn;
            // the split tape holds 3 T B H pieces, past 2^32 for the largest admitted shapes
            const u64 pc = (t * B + b) * 3 * H + h;
            split3(gsyn, g3[pc], g3[pc + H], g3[pc + 2 * H]);
        }
        const uint32_t prev = (uint32_t)((tp * B + b) * H + h);
        ngr = gs_read[prev];
        nsp = spikes[prev];
        nmt = mem_tape[prev];
    };
    auto update = [&]() {
        const float qq = slope * fabsf(mt - theta) + 1.0f;
        const float sigma = 1.0f / (qq * qq);
        const float gs = gr + rec;
        const float gm_next = gmem, gs_next = gsyn;
        gmem = beta * (1.0f - sp) * gm_next + gs * sigma;
        gsyn = (1.0f - sp) * gm_next + alpha * gs_next;
        gr = ngr;
        sp = nsp;
        mt = nmt;
    };
    emit(T - 1);
    for (u64 t = T; t-- > 0;) {
        lds_barrier();
        float p = 0.0f;
        if (t > 0) {
            p = quad_sum(quarter_dot(xs[t & 1], w, q));
            update();
            emit(t - 1);
        } else {
            update();
        }
        rec = p;
    }
}

// ------------------------------------- three ticks per exchange (H = 256, one sample per workgroup)
// The recurrent product of tick t enters the membrane three ticks later at the earliest: P_t =
// s_t W_rec enters h1_{t+1}, hence syn_{t+2}, hence mem_{t+3} and s_{t+3} (the membrane update
// reads the synaptic current of the tick before).  So once s_t0, s_t0+1 and s_t0+2 are known the
// products of those three ticks form one 3-row product, and the updates that follow give s_t0+3
// .. s_t0+5: one exchange (two workgroup barriers) per three ticks instead of three.  The backward
// pass has the same three-tick latency (Q_t = g_t W_rec^T enters gmem_{t-1}, hence gsyn_{t-2}).
//
// The 3-row product runs on v_mfma_f32_4x4x1f32 (16 blocks of 4 x 4, K = 1; row 3 is zero):
// wave w takes the 64 columns 64 (w % 4) .. + 63 (lane l: column 64 (w % 4) + l) over the
// quarter of the rows 64 (w / 4) .. + 63, whose weights it keeps in 64 registers as B operands.
// The A operand is broadcast from one block (CBSZ = 4, ABID = b): lane 4b + i holds row i's value
// x_i[64 (w / 4) + 16 r + b] in register r, one 16-byte LDS read per lane per exchange.  Each
// wave accumulates row k into accumulator k % 4 in ascending k and sums them as
// (a0 + a1) + (a2 + a3); the four quarters' partial products meet in LDS and are summed as
// (q0 + q1) + (q2 + q3): the order of the one-tick passes above (quarter_dot, quad_sum), so with
// the MFMA's fused multiply-add per element both give the same bits.  The four waves of a column
// update its state redundantly (identical bits); the first quarter's writes the tapes and the
// exchanged values.
constexpr int TRI_ROWS = 3;

// x_i[k] of the exchanged 4 x 256 operand (i = tick row, k = hidden unit) in the A-register layout
__device__ __forceinline__ int tri_at(int k, int i) {
    const int m = k & 63;
    return (k >> 6) * 256 + ((m & 15) * 4 + i) * 4 + (m >> 4);
}

// Rows M .. M + 3 of the wave's quarter (row 64 kq + m: A register m / 16, broadcast block m % 16,
// accumulator m % 4), then the rest.
template <int M>
__device__ __forceinline__ void tri_chain(const float4_t& a, const float* w, float4_t* acc) {
    if constexpr (M < 64) {
        acc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[M / 16], w[M], acc[0], 4, M % 16, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[M / 16], w[M + 1], acc[1], 4, M % 16 + 1, 0);
        acc[2] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[M / 16], w[M + 2], acc[2], 4, M % 16 + 2, 0);
        acc[3] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[M / 16], w[M + 3], acc[3], 4, M % 16 + 3, 0);
        tri_chain<M + 4>(a, w, acc);
    }
}

// The wave's quarter (rows 64 kq .. 64 kq + 63) of the 4-row product for its lane's column.
__device__ __forceinline__ float4_t tri_quarter(const float* __restrict__ x, const float* w, unsigned lane,
                                                unsigned kq) {
    const float4_t a = *reinterpret_cast<const float4_t*>(x + kq * 256 + lane * 4);
    float4_t acc[4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f},
                       {0.0f, 0.0f, 0.0f, 0.0f}};
    tri_chain<0>(a, w, acc);
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// The lane's column of the 4-row product from the four quarters' partial products in LDS.
__device__ __forceinline__ float4_t tri_sum(const float4_t* part, unsigned h) {
    return (part[h] + part[VEC_H + h]) + (part[2 * VEC_H + h] + part[3 * VEC_H + h]);
}

// Forward pass, three ticks per exchange.  Before block t0 (t0 = 0, 3, ...) the exchange holds
// s_t0, s_t0+1, s_t0+2 and the first quarter's lanes hold syn_t0+1, mem_t0+2 and s_t0+2 of their
// columns; the block forms P_t0 .. P_t0+2 and those lanes run, for j = 0, 1, 2, the current update
// of tick t0 + 1 + j (syn_t0+2+j = alpha syn + Hin_t0+1+j + P_t0+j) and the membrane update of
// tick t0 + 2 + j (mem_t0+3+j = (beta mem + syn_t0+2+j) (1 - s_t0+2+j)) and write the tapes: the
// operations of forward_vec's tick loop, in the same order per value.  The second quarter's waves
// load the block's inputs and stage them in LDS, so that the updating lanes never wait for a load
// (a wait for a load also waits for every store issued before it).
__global__ void __launch_bounds__(1024) forward_tri(u64 T, u64 B, float alpha, float beta, float theta,
                                                    const float* __restrict__ w_rec, const float* __restrict__ hin,
                                                    float* __restrict__ mem_tape, float* __restrict__ spikes,
                                                    bf16_t* __restrict__ spikes16) {
    constexpr u64 H = VEC_H;
    __shared__ __attribute__((aligned(16))) float xs[2][4 * 256];
    __shared__ float4_t part[4 * H];
    __shared__ float ins[TRI_ROWS][H];   // the block's inputs Hin_t0+1 .. Hin_t0+3
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64, kq = wave >> 2;
    const unsigned h = (wave & 3u) * 64u + lane;
    const u64 b = blockIdx.x;
    const bool first = kq == 0, loader = kq == 1;
    float w[64];
#pragma unroll
    for (int m = 0; m < 64; ++m) w[m] = w_rec[(64 * kq + m) * H + h];
    // the weights are waited for here: otherwise the compiler's wait counting assumes they may
    // still be pending in every block and waits in the middle of the product for the block's
    // other memory accesses
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    for (unsigned j = threadIdx.x; j < 2 * 4 * 256; j += 1024) (&xs[0][0])[j] = 0.0f;   // row 3 stays zero
    lds_barrier();
    auto input = [&](u64 t) { return hin[(uint32_t)(((t < T ? t : T - 1) * B + b) * H + h)]; };
    // s_t of the membrane entering tick t, taped and exchanged in row `row` of buffer `x` (`full`:
    // t is known to lie inside the run)
    auto emit = [&](u64 t, float mem, float* x, int row, bool full) {
        const float s = mem > theta ? 1.0f : 0.0f;
        x[tri_at((int)h, row)] = s;
        if (full || t < T) {
            const uint32_t at = (uint32_t)((t * B + b) * H + h);
            mem_tape[at] = mem;
            spikes[at] = s;
            spikes16[at] = s != 0.0f ? (bf16_t)0x3F80 : (bf16_t)0;
        }
        return s;
    };
    float syn = 0.0f, mem = 0.0f, s = 0.0f;
    if (first) {
        // ticks 0 .. 2 need no product (P_-1 = 0 enters syn_1, nothing enters mem_1 or mem_2)
        s = emit(0, mem, xs[0], 0, false);
        const float h1 = input(0) + 0.0f;
        const float sy = syn;
        syn = alpha * sy + h1;                    // syn_1
        mem = (beta * mem + sy) * (1.0f - s);     // mem_1
        s = emit(1, mem, xs[0], 1, false);
        mem = (beta * mem + syn) * (1.0f - s);    // mem_2
        s = emit(2, mem, xs[0], 2, false);
    }
    // block k (t0 = 3 k); `full`: its three taped ticks t0 + 3 .. t0 + 5 lie inside the run, so the
    // update runs without a branch
    auto block = [&](u64 t0, u64 k, bool full) {
        float in[TRI_ROWS] = {0.0f, 0.0f, 0.0f};
        if (loader)
#pragma unroll
            for (int j = 0; j < TRI_ROWS; ++j) in[j] = input(t0 + 1 + j);
        lds_barrier();
        part[kq * VEC_H + h] = tri_quarter(xs[k & 1], w, lane, kq);
        // every wave's global accesses complete here, under the other waves' products: the
        // loading waves' inputs, and the updating lanes' tape stores of the block before (their
        // registers are then free for the update without a wait on its chain)
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        if (loader)
#pragma unroll
            for (int j = 0; j < TRI_ROWS; ++j) ins[j][h] = in[j];
        lds_barrier();
        if (first) {
            const float4_t p = tri_sum(part, h);
            float* next = xs[(k + 1) & 1];
#pragma unroll
            for (int j = 0; j < TRI_ROWS; ++j) {
                const float h1 = ins[j][h] + p[j];
                const float sy = syn;
                syn = alpha * sy + h1;                 // syn_t0+2+j
                mem = (beta * mem + syn) * (1.0f - s); // mem_t0+3+j
                s = emit(t0 + 3 + j, mem, next, j, full);
            }
        }
    };
    u64 t0 = 0, k = 0;
    for (; t0 + 5 < T; t0 += 3, ++k) block(t0, k, true);
    for (; t0 + 3 < T; t0 += 3, ++k) block(t0, k, false);
}

// Backward pass, three ticks per exchange, descending.  Before block t0 (t0 = T - 1, T - 4, ...)
// the exchange holds g_t0, g_t0-1, g_t0-2 (g_t = gsyn_t+1, the adjoint of syn_t+1) and the first
// quarter's lanes hold gmem_t0 and gsyn_t0-1 of their columns; the block forms Q_t0 .. Q_t0-2 and
// those lanes run, for j = 0, 1, 2, the membrane adjoint of tick t0 - 1 - j (gmem = beta (1 - s)
// gmem + (gs_read + Q_t0-j) sigma) and the current adjoint of tick t0 - 2 - j (gsyn = (1 - s) gmem
// + alpha gsyn), whose value is g_t0-3-j: backward_vec's operations, in the same order per value.
// As in the forward pass, the second quarter's waves load and stage the block's tape values; they
// also form beta (1 - s), sigma and 1 - s from them (the same operations, off the updating lanes'
// chain) after their share of the product, so that no barrier waits for the loads.  The updating
// lanes leave g in LDS (double-buffered by block parity) and the third quarter's waves write it,
// and its split pieces, in the next block while its update runs (measured faster for this pass
// than the updating lanes' own stores, which the forward pass keeps).
__global__ void __launch_bounds__(1024) backward_tri(u64 T, u64 B, float alpha, float beta, float theta, float slope,
                                                     const float* __restrict__ w_rec,
                                                     const float* __restrict__ gs_read,
                                                     const float* __restrict__ mem_tape,
                                                     const float* __restrict__ spikes, float* __restrict__ g1,
                                                     bf16_t* __restrict__ g3) {
    constexpr u64 H = VEC_H;
    __shared__ __attribute__((aligned(16))) float xs[2][4 * 256];
    __shared__ float4_t part[4 * H];
    // the block's gs_read, beta (1 - s) and sigma of ticks t0 - 1 - j, 1 - s of ticks t0 - 2 - j
    __shared__ float tin[4][TRI_ROWS][H];
    __shared__ float tout[2][TRI_ROWS][H];   // g_t0-3-j of the block, by parity
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64, kq = wave >> 2;
    const unsigned h = (wave & 3u) * 64u + lane;
    const u64 b = blockIdx.x;
    const bool first = kq == 0, loader = kq == 1, storer = kq == 2;
    float w[64];
#pragma unroll
    for (int m = 0; m < 64; ++m) w[m] = w_rec[(u64)h * H + 64 * kq + m];   // row h of W_rec: column h of W_rec^T
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): as in the forward pass
    for (unsigned j = threadIdx.x; j < 2 * 4 * 256; j += 1024) (&xs[0][0])[j] = 0.0f;
    lds_barrier();
    auto at = [&](i64 t) { return (uint32_t)(((u64)(t > 0 ? t : 0) * B + b) * H + h); };
    auto write = [&](i64 t, float g) {
        if (t >= 0) {
            g1[at(t)] = g;
            const u64 pc = ((u64)t * B + b) * 3 * H + h;
            split3(g, g3[pc], g3[pc + H], g3[pc + 2 * H]);
        }
    };
    auto sigma_of = [&](float mt) {
        const float qq = slope * fabsf(mt - theta) + 1.0f;
        return 1.0f / (qq * qq);
    };
    const i64 last = (i64)T - 1;
    float gmem = 0.0f, gsyn = 0.0f;
    if (first) {
        // g_T-1 = gsyn_T = 0; g_T-2 and g_T-3 need no product (Q_T = 0)
        xs[0][tri_at((int)h, 0)] = gsyn;
        write(last, gsyn);
        const float gr = gs_read[at(last)], sp = spikes[at(last)], sigma = sigma_of(mem_tape[at(last)]);
        const float sp1 = spikes[at(last - 1)];
        const float gs = gr + 0.0f;
        const float gm_next = gmem, gs_next = gsyn;
        gmem = beta * (1.0f - sp) * gm_next + gs * sigma;   // gmem_T-1
        gsyn = (1.0f - sp) * gm_next + alpha * gs_next;     // gsyn_T-1 = g_T-2
        xs[0][tri_at((int)h, 1)] = gsyn;
        write(last - 1, gsyn);
        gsyn = (1.0f - sp1) * gmem + alpha * gsyn;          // gsyn_T-2 = g_T-3
        xs[0][tri_at((int)h, 2)] = gsyn;
        write(last - 2, gsyn);
        // the compiler's wait counting then knows these stores complete before the loop
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    }
    // the written ticks t0 - 3 .. t0 - 5 of block k, from LDS
    auto store_block = [&](i64 t0, i64 k) {
#pragma unroll
        for (int j = 0; j < TRI_ROWS; ++j) write(t0 - 3 - j, tout[k & 1][j][h]);
    };
    auto block = [&](i64 t0, i64 k) {
        float v[4][TRI_ROWS];   // not initialised: see forward_tri's inputs
        if (loader)
#pragma unroll
            for (int j = 0; j < TRI_ROWS; ++j) {
                v[0][j] = gs_read[at(t0 - 1 - j)];
                v[1][j] = spikes[at(t0 - 1 - j)];
                v[2][j] = mem_tape[at(t0 - 1 - j)];
                v[3][j] = spikes[at(t0 - 2 - j)];
            }
        lds_barrier();
        part[kq * VEC_H + h] = tri_quarter(xs[k & 1], w, lane, kq);
        if (loader)
#pragma unroll
            for (int j = 0; j < TRI_ROWS; ++j) {
                // the loads are waited for here, after the product, and the derived values formed
                tin[0][j][h] = v[0][j];
                tin[1][j][h] = beta * (1.0f - v[1][j]);
                tin[2][j][h] = sigma_of(v[2][j]);
                tin[3][j][h] = 1.0f - v[3][j];
            }
        lds_barrier();
        if (first) {
            const float4_t q = tri_sum(part, h);
            float* next = xs[(k + 1) & 1];
#pragma unroll
            for (int j = 0; j < TRI_ROWS; ++j) {
                const float gs = tin[0][j][h] + q[j];
                gmem = tin[1][j][h] * gmem + gs * tin[2][j][h];   // gmem_t0-1-j
                gsyn = tin[3][j][h] * gmem + alpha * gsyn;        // gsyn_t0-2-j = g_t0-3-j
                next[tri_at((int)h, j)] = gsyn;
                tout[k & 1][j][h] = gsyn;
            }
        }
        if (storer && k > 0) store_block(t0 + 3, k - 1);
    };
    i64 t0 = last, k = 0;
    for (; t0 - 3 >= 0; t0 -= 3, ++k) block(t0, k);
    lds_barrier();
    if (storer && k > 0) store_block(t0 + 3, k - 1);
}

// --------------------------------------------------------------- readout
// Per (sample, class): F, U recurrence over the ticks, logits = max(U_0 .. U_T)
// and the tick whose update produced it (-1: the initial zero).
__global__ void readout_forward(u64 T, u64 B, u64 C, float alpha, float beta, const float* __restrict__ h2,
                                float* __restrict__ logits, int* __restrict__ argmax) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= B * C) return;
    float f = 0.0f, u = 0.0f, best = 0.0f;
    int arg = -1;
#pragma unroll 10
    for (u64 t = 0; t < T; ++t) {
        const float u_next = beta * u + f;
        f = alpha * f + h2[t * B * C + x];
        u = u_next;
        if (u > best) {
            best = u;
            arg = (int)t;
        }
    }
    logits[x] = best;
    argmax[x] = arg;
}

// Cross-entropy of one sample and the logit adjoint (softmax - onehot) / B: one wavefront per
// sample, lanes over classes; max and sum by xor butterflies (commutative steps, so every lane
// ends with the same bits).  Grid: ceil(B / 4) workgroups of 256.
__global__ void __launch_bounds__(256) loss_kernel(u64 B, u64 C, const float* __restrict__ logits,
                                                   const u64* __restrict__ labels, float* __restrict__ losses,
                                                   float* __restrict__ glogit) {
    const unsigned lane = threadIdx.x % 64;
    const u64 b = (u64)blockIdx.x * 4 + threadIdx.x / 64;
    if (b >= B) return;
    const float* z = logits + b * C;
    float top = -__builtin_huge_valf();
    for (u64 c = lane; c < C; c += 64) top = fmaxf(top, z[c]);
    for (int o = 32; o > 0; o >>= 1) top = fmaxf(top, __shfl_xor(top, o));
    float denom = 0.0f;
    for (u64 c = lane; c < C; c += 64) denom += atlas_expf(z[c] - top);
    for (int o = 32; o > 0; o >>= 1) denom += __shfl_xor(denom, o);
    const u64 label = labels[b];
    if (lane == 0) losses[b] = top + atlas_logf(denom) - z[label];
    for (u64 c = lane; c < C; c += 64)
        glogit[b * C + c] = (atlas_expf(z[c] - top) / denom - (c == label ? 1.0f : 0.0f)) / (float)B;
}

// Adjoint of the readout recurrence: gh2_t = adjoint of F_{t+1}.
__global__ void readout_backward(u64 T, u64 B, u64 C, float alpha, float beta, const float* __restrict__ glogit,
                                 const int* __restrict__ argmax, float* __restrict__ gh2) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= B * C) return;
    float gu = 0.0f, gf = 0.0f;
    const int arg = argmax[x];
    const float direct = glogit[x];
    for (u64 t = T; t-- > 0;) {
        if ((int)t == arg) gu += direct;
        gh2[t * B * C + x] = gf;
        const float gu_prev = beta * gu;
        gf = gu + alpha * gf;
        gu = gu_prev;
    }
}

// ---------------------------------------------------------------- helpers
__global__ void fill(float* __restrict__ p, u64 n, float value) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x < n) p[x] = value;
}

// out[m][c] = sum over split s and piece p of partials[s][m][p * cols + c], s then p ascending
// (a fixed order: deterministic).  pieces = 1 for a float32 product.
__global__ void reduce_partials(u64 rows, u64 cols, u64 splits, u64 pieces, const float* __restrict__ partials,
                                float* __restrict__ out) {
    const u64 e = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= rows * cols) return;
    const u64 m = e / cols, c = e % cols, n = rows * cols * pieces, terms = splits * pieces;
    const float* base = partials + m * pieces * cols + c;
    float sum = 0.0f;
#pragma unroll 8
    for (u64 j = 0; j < terms; ++j) sum += base[(j / pieces) * n + (j % pieces) * cols];
    out[e] = sum;
}

// x is given sample-major (b, t, i); rows of the GEMMs are (t, b).  Also writes x3, the rows
// in bfloat16 repeated three times ([x | x | x], the A operand against the three stacked pieces
// of W_in), and clears *exact if some value is not a bfloat16.
__global__ void to_tick_major(u64 B, u64 T, u64 I, const float* __restrict__ src, float* __restrict__ dst,
                              bf16_t* __restrict__ x3, int* __restrict__ exact) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= B * T * I) return;
    const u64 i = x % I, t = (x / I) % T, b = x / (I * T);
    const float v = src[x];
    const u64 row = t * B + b;
    dst[row * I + i] = v;
    const bf16_t q = to_bf16(v);
    if (from_bf16(q) != v) *exact = 0;
    x3[row * 3 * I + i] = q;
    x3[row * 3 * I + I + i] = q;
    x3[row * 3 * I + 2 * I + i] = q;
}

// Three bfloat16 pieces of W (rows x cols) stacked along the rows: [W_hi; W_mid; W_lo].
__global__ void split_rows(u64 n, const float* __restrict__ w, bf16_t* __restrict__ w3) {
    const u64 e = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    split3(w[e], w3[e], w3[n + e], w3[2 * n + e]);
}

__global__ void fill_int(int* __restrict__ p, int value) { *p = value; }

__global__ void adam(u64 n, float* __restrict__ w, float* __restrict__ m, float* __restrict__ v,
                     const float* __restrict__ g, float lr, float beta1, float beta2, float eps, float bc1, float bc2) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n) return;
    const float grad = g[x];
    const float m1 = beta1 * m[x] + (1.0f - beta1) * grad;
    const float v1 = beta2 * v[x] + (1.0f - beta2) * grad * grad;
    m[x] = m1;
    v[x] = v1;
    w[x] -= lr * (m1 / bc1) / (sqrtf(v1 / bc2) + eps);
}

}  // namespace

struct AtlasRsnn {
    AtlasRsnnSpec spec{};
    int device = 0;
    hipStream_t stream = nullptr;
    rocblas_handle blas = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    hipEvent_t marks[ATLAS_RSNN_PHASES + 1] = {};
    bool profiling = false;
    // H = 256: the one-tick passes (forward_vec, backward_vec) instead of three ticks per exchange,
    // chosen at creation by ATLAS_RSNN_PASSES=vec (both give the same bits)
    bool one_tick = false;
    u64 step_count = 0;
    float* w[3] = {};      // W_in (I x H), W_rec (H x H), W_out (H x C): row-major (source, target)
    float* m[3] = {};
    float* v[3] = {};
    float* g[3] = {};
    u64 size[3] = {};
    float *x = nullptr, *hin = nullptr, *syn = nullptr, *mem = nullptr, *mem_tape = nullptr, *spikes = nullptr;
    float *h2 = nullptr, *logits = nullptr, *losses = nullptr, *glogit = nullptr, *gh2 = nullptr;
    float *gs_read = nullptr, *gmem = nullptr, *gsyn = nullptr, *g1 = nullptr, *staging = nullptr;
    float* partials = nullptr;  // split-K partial products of the weight gradients
    // bfloat16 operands of the split-precision GEMMs: x3 = [x | x | x] rows, the spike tape,
    // g3 = [g_hi | g_mid | g_lo] rows of the syn adjoint, w3_in = [W_hi; W_mid; W_lo]
    bf16_t *x3 = nullptr, *spikes16 = nullptr, *g3 = nullptr, *w3_in = nullptr;
    int* exact = nullptr;
    bool binary_inputs = false;  // every input value of the batch is a bfloat16
    int* argmax = nullptr;
    u64* labels = nullptr;
    bool has_batch = false;
    double last_ms = 0.0;

    ~AtlasRsnn() {
        for (int k = 0; k < 3; ++k)
            for (float* p : {w[k], m[k], v[k], g[k]})
                if (p) (void)hipFree(p);
        for (void* p : {(void*)x, (void*)hin, (void*)syn, (void*)mem, (void*)mem_tape, (void*)spikes, (void*)h2,
                        (void*)logits, (void*)losses, (void*)glogit, (void*)gh2, (void*)gs_read, (void*)gmem,
                        (void*)gsyn, (void*)g1, (void*)staging, (void*)partials, (void*)argmax, (void*)labels,
                        (void*)x3, (void*)spikes16, (void*)g3, (void*)w3_in, (void*)exact})
            if (p) (void)hipFree(p);
        if (blas) (void)rocblas_destroy_handle(blas);
        for (hipEvent_t e : marks)
            if (e) (void)hipEventDestroy(e);
        if (start) (void)hipEventDestroy(start);
        if (stop) (void)hipEventDestroy(stop);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

// Row-major C(MxN) = op(A) op(B) + beta C through column-major rocBLAS (C^T = op(B)^T op(A)^T).
bool gemm(AtlasRsnn* r, bool ta, bool tb, u64 M, u64 N, u64 K, const float* A, u64 lda, const float* Bm, u64 ldb,
          float* Cm, u64 ldc, float beta = 0.0f) {
    const float one = 1.0f;
    return rocblas_sgemm(r->blas, tb ? rocblas_operation_transpose : rocblas_operation_none,
                         ta ? rocblas_operation_transpose : rocblas_operation_none, (rocblas_int)N, (rocblas_int)M,
                         (rocblas_int)K, &one, Bm, (rocblas_int)ldb, A, (rocblas_int)lda, &beta, Cm,
                         (rocblas_int)ldc) == rocblas_status_success;
}

// Largest hidden size served by the persistent passes (the W_rec slab lives in registers);
// beyond it every tick is a launch of the tiled kernels.
constexpr u64 PERSISTENT_MAX_HIDDEN = 256;

template <int KMAX, int KREG, bool FULL>
void launch_passes(AtlasRsnn* r, bool forward) {
    const AtlasRsnnSpec& s = r->spec;
    const dim3 grid((unsigned)(s.batch / 4)), block(KMAX);
    if (forward)
        hipLaunchKernelGGL((forward_pass<KMAX, KREG, FULL>), grid, block, 0, r->stream, s.time, s.batch, s.hidden,
                           s.alpha, s.beta, s.threshold, r->w[1], r->hin, r->mem_tape, r->spikes, r->spikes16);
    else
        hipLaunchKernelGGL((backward_pass<KMAX, KREG, FULL>), grid, block, 0, r->stream, s.time, s.batch, s.hidden,
                           s.alpha, s.beta, s.threshold, s.slope, r->w[1], r->gs_read, r->mem_tape, r->spikes, r->g1,
                           r->g3);
}

// H = 256 (configuration 4): one sample per workgroup; otherwise four samples per workgroup with
// the slab's rows in registers, all of them up to 128, between 129 and 255 192 in registers and
// 64 in LDS.
void persistent_pass(AtlasRsnn* r, bool forward) {
    const u64 H = r->spec.hidden;
    if (H == 256) {
        const AtlasRsnnSpec& s = r->spec;
        if (forward)
            hipLaunchKernelGGL(r->one_tick ? forward_vec : forward_tri, dim3((unsigned)s.batch), dim3(1024), 0,
                               r->stream, s.time, s.batch, s.alpha, s.beta, s.threshold, r->w[1], r->hin, r->mem_tape,
                               r->spikes, r->spikes16);
        else
            hipLaunchKernelGGL(r->one_tick ? backward_vec : backward_tri, dim3((unsigned)s.batch), dim3(1024), 0,
                               r->stream, s.time, s.batch, s.alpha, s.beta, s.threshold, s.slope, r->w[1], r->gs_read,
                               r->mem_tape, r->spikes, r->g1, r->g3);
    } else if (H <= 64) launch_passes<64, 64, false>(r, forward);
    else if (H <= 128) launch_passes<128, 128, false>(r, forward);
    else launch_passes<256, 192, false>(r, forward);
}

// Phase boundaries of one step, recorded only by atlas_rsnn_profile.
void mark(AtlasRsnn* r, int phase) {
    if (r->profiling) (void)hipEventRecord(r->marks[phase], r->stream);
}

// Strided-batched form of gemm(): batch k multiplies the k-th block of rows.
bool gemm_batched(AtlasRsnn* r, bool ta, bool tb, u64 M, u64 N, u64 K, const float* A, u64 lda, u64 stride_a,
                  const float* Bm, u64 ldb, u64 stride_b, float* Cm, u64 ldc, u64 stride_c, u64 batch) {
    const float one = 1.0f, zero = 0.0f;
    return rocblas_sgemm_strided_batched(r->blas, tb ? rocblas_operation_transpose : rocblas_operation_none,
                                         ta ? rocblas_operation_transpose : rocblas_operation_none, (rocblas_int)N,
                                         (rocblas_int)M, (rocblas_int)K, &one, Bm, (rocblas_int)ldb,
                                         (rocblas_stride)stride_b, A, (rocblas_int)lda, (rocblas_stride)stride_a, &zero,
                                         Cm, (rocblas_int)ldc, (rocblas_stride)stride_c,
                                         (rocblas_int)batch) == rocblas_status_success;
}

// Chunks of (tick, sample) rows for a weight gradient: the output has few tiles and the
// reduction over rows is long, so the rows are split and the partials summed afterwards.  16
// chunks of >= 1024 rows give the GEMM a few hundred workgroups while the partials the
// reduction reads stay a small multiple of the output.
constexpr u64 MAX_SPLITS = 16;

u64 splits_for(u64 rows) {
    for (u64 k = MAX_SPLITS; k > 1; k /= 2)
        if (rows % k == 0 && rows / k >= 1024) return k;
    return 1;
}

// C(M x N) = A^T B over `rows` rows: A is rows x M (row-major, lda), B rows x N (ldb).
bool gradient(AtlasRsnn* r, u64 M, u64 N, u64 rows, const float* A, u64 lda, const float* Bm, u64 ldb, float* C) {
    const u64 k = splits_for(rows);
    if (k == 1) return gemm(r, true, false, M, N, rows, A, lda, Bm, ldb, C, N);
    const u64 chunk = rows / k;
    if (!gemm_batched(r, true, false, M, N, chunk, A, lda, chunk * lda, Bm, ldb, chunk * ldb, r->partials, N, M * N, k))
        return false;
    hipLaunchKernelGGL(reduce_partials, dim3(blocks(M * N)), dim3(256), 0, r->stream, M, N, k, (u64)1, r->partials, C);
    return true;
}

// Row-major C(M x N) = A(M x K) B(K x N) with bfloat16 operands, float32 accumulation and output.
bool gemm_bf16(AtlasRsnn* r, u64 M, u64 N, u64 K, const bf16_t* A, u64 lda, const bf16_t* Bm, u64 ldb, float* Cm,
               u64 ldc) {
    const float one = 1.0f, zero = 0.0f;
    return rocblas_gemm_ex(r->blas, rocblas_operation_none, rocblas_operation_none, (rocblas_int)N, (rocblas_int)M,
                           (rocblas_int)K, &one, Bm, rocblas_datatype_bf16_r, (rocblas_int)ldb, A,
                           rocblas_datatype_bf16_r, (rocblas_int)lda, &zero, Cm, rocblas_datatype_f32_r,
                           (rocblas_int)ldc, Cm, rocblas_datatype_f32_r, (rocblas_int)ldc, rocblas_datatype_f32_r,
                           rocblas_gemm_algo_standard, 0, 0) == rocblas_status_success;
}

// C(M x H) = A^T G over `rows` rows from bfloat16 operands: A (rows x M, lda) exactly
// representable, G3 (rows x 3H) the three pieces of G.  Split over chunks of rows; the partials
// are summed over chunks and pieces.
bool gradient_split(AtlasRsnn* r, u64 M, u64 H, u64 rows, const bf16_t* A, u64 lda, const bf16_t* g3, float* C) {
    const u64 k = splits_for(rows), chunk = rows / k, N = 3 * H;
    const float one = 1.0f, zero = 0.0f;
    if (rocblas_gemm_strided_batched_ex(
            r->blas, rocblas_operation_none, rocblas_operation_transpose, (rocblas_int)N, (rocblas_int)M,
            (rocblas_int)chunk, &one, g3, rocblas_datatype_bf16_r, (rocblas_int)N, (rocblas_stride)(chunk * N), A,
            rocblas_datatype_bf16_r, (rocblas_int)lda, (rocblas_stride)(chunk * lda), &zero, r->partials,
            rocblas_datatype_f32_r, (rocblas_int)N, (rocblas_stride)(M * N), r->partials, rocblas_datatype_f32_r,
            (rocblas_int)N, (rocblas_stride)(M * N), (rocblas_int)k, rocblas_datatype_f32_r,
            rocblas_gemm_algo_standard, 0, 0) != rocblas_status_success)
        return false;
    hipLaunchKernelGGL(reduce_partials, dim3(blocks(M * H)), dim3(256), 0, r->stream, M, H, k, (u64)3, r->partials, C);
    return true;
}

int run_step(AtlasRsnn* r, bool train, char* err, size_t cap) {
    const AtlasRsnnSpec& s = r->spec;
    const u64 B = s.batch, T = s.time, I = s.inputs, H = s.hidden, C = s.classes;
    hipStream_t st = r->stream;
    const unsigned tick_blocks = (unsigned)(((B / 16) * (H / 16) + 3) / 4);
    const bool persistent = H <= PERSISTENT_MAX_HIDDEN;
    mark(r, 0);
    // split-precision bfloat16 GEMMs where one operand is exactly representable: the spike tape
    // always (written by the persistent passes), the inputs when every value is a bfloat16
    const bool split_rec = persistent, split_in = persistent && r->binary_inputs;
    // forward: input projection for every tick at once
    if (split_in) {
        if (!gemm_bf16(r, T * B, H, 3 * I, r->x3, 3 * I, r->w3_in, H, r->hin, H))
            return fail(err, cap, 4, "rocBLAS x3 W3_in");
    } else if (!gemm(r, false, false, T * B, H, I, r->x, I, r->w[0], H, r->hin, H)) {
        return fail(err, cap, 4, "rocBLAS x W_in");
    }
    if (!persistent) {
        hipLaunchKernelGGL(fill, dim3(blocks(B * H)), dim3(256), 0, st, r->syn, B * H, 0.0f);
        hipLaunchKernelGGL(fill, dim3(blocks(B * H)), dim3(256), 0, st, r->mem, B * H, 0.0f);
    }
    mark(r, 1);
    if (persistent)
        persistent_pass(r, true);
    else
        for (u64 t = 0; t < T; ++t)
            hipLaunchKernelGGL(forward_tick, dim3(tick_blocks), dim3(256), 0, st, t, B, H, s.alpha, s.beta,
                               s.threshold, r->w[1], r->hin, r->syn, r->mem, r->mem_tape, r->spikes);
    mark(r, 2);
    if (!gemm(r, false, false, T * B, C, H, r->spikes, H, r->w[2], C, r->h2, C)) return fail(err, cap, 4, "rocBLAS S W_out");
    hipLaunchKernelGGL(readout_forward, dim3(blocks(B * C)), dim3(256), 0, st, T, B, C, s.alpha, s.beta, r->h2,
                       r->logits, r->argmax);
    hipLaunchKernelGGL(loss_kernel, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, st, B, C, r->logits, r->labels,
                       r->losses, r->glogit);
    mark(r, 3);
    if (train) {
        hipLaunchKernelGGL(readout_backward, dim3(blocks(B * C)), dim3(256), 0, st, T, B, C, s.alpha, s.beta,
                           r->glogit, r->argmax, r->gh2);
        if (!gemm(r, false, true, T * B, H, C, r->gh2, C, r->w[2], C, r->gs_read, H))
            return fail(err, cap, 4, "rocBLAS gh2 W_out^T");
        if (!persistent) {
            hipLaunchKernelGGL(fill, dim3(blocks(B * H)), dim3(256), 0, st, r->gmem, B * H, 0.0f);
            hipLaunchKernelGGL(fill, dim3(blocks(B * H)), dim3(256), 0, st, r->gsyn, B * H, 0.0f);
        }
        mark(r, 4);
        if (persistent)
            persistent_pass(r, false);
        else
            for (u64 t = T; t-- > 0;)
                hipLaunchKernelGGL(backward_tick, dim3(tick_blocks), dim3(256), 0, st, t, T, B, H, s.alpha, s.beta,
                                   s.threshold, s.slope, r->w[1], r->gs_read, r->mem_tape, r->spikes, r->gmem,
                                   r->gsyn, r->g1);
        mark(r, 5);
        // weight gradients over every (tick, sample) row
        if (split_in ? !gradient_split(r, I, H, T * B, r->x3, 3 * I, r->g3, r->g[0])
                     : !gradient(r, I, H, T * B, r->x, I, r->g1, H, r->g[0]))
            return fail(err, cap, 4, "rocBLAS dW_in");
        if (T > 1 && (split_rec ? !gradient_split(r, H, H, (T - 1) * B, r->spikes16, H, r->g3 + B * 3 * H, r->g[1])
                                : !gradient(r, H, H, (T - 1) * B, r->spikes, H, r->g1 + B * H, H, r->g[1])))
            return fail(err, cap, 4, "rocBLAS dW_rec");
        if (T == 1) hipLaunchKernelGGL(fill, dim3(blocks(H * H)), dim3(256), 0, st, r->g[1], H * H, 0.0f);
        if (!gradient(r, H, C, T * B, r->spikes, H, r->gh2, C, r->g[2])) return fail(err, cap, 4, "rocBLAS dW_out");
        mark(r, 6);
        r->step_count += 1;
        const float bc1 = (float)(1.0 - std::pow((double)s.beta1, (double)r->step_count));
        const float bc2 = (float)(1.0 - std::pow((double)s.beta2, (double)r->step_count));
        if (s.learning_rate != 0.0f)
            for (int k = 0; k < 3; ++k)
                hipLaunchKernelGGL(adam, dim3(blocks(r->size[k])), dim3(256), 0, st, r->size[k], r->w[k], r->m[k],
                                   r->v[k], r->g[k], s.learning_rate, s.beta1, s.beta2, s.epsilon, bc1, bc2);
        if (s.learning_rate != 0.0f)
            hipLaunchKernelGGL(split_rows, dim3(blocks(I * H)), dim3(256), 0, st, I * H, r->w[0], r->w3_in);
        mark(r, 7);
    }
    if (hipGetLastError() != hipSuccess) return fail(err, cap, 4, "kernel launch failed");
    return 0;
}

}  // namespace

extern "C" {

int atlas_rsnn_create(const AtlasRsnnSpec* spec, const float* w_in, const float* w_rec, const float* w_out,
                      AtlasRsnn** out, char* err, size_t cap) {
    try {
        if (!spec || !w_in || !w_rec || !w_out || !out) return fail(err, cap, 7, "null argument");
        *out = nullptr;
        const AtlasRsnnSpec& s = *spec;
        if (!s.batch || !s.time || !s.inputs || !s.hidden || !s.classes || s.batch % 16 || s.hidden % 16)
            return fail(err, cap, 7, "batch and hidden must be positive multiples of 16");
        if (s.batch * s.time * (s.inputs > s.hidden ? s.inputs : s.hidden) > (1ull << 31))
            return fail(err, cap, 7, "batch x time x width exceeds the GEMM index range");
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count < 1) return fail(err, cap, 1, "no HIP GPU");
        int device = 0;
        if (const char* choice = getenv("B2_TRAIN_HIP_DEVICE")) device = atoi(choice);
        if (device < 0 || device >= count || hipSetDevice(device) != hipSuccess)
            return fail(err, cap, 1, "invalid B2_TRAIN_HIP_DEVICE");
        AtlasRsnn* r = new (std::nothrow) AtlasRsnn();
        if (!r) return fail(err, cap, 7, "host allocation failed");
        r->spec = s;
        r->device = device;
        if (const char* passes = getenv("ATLAS_RSNN_PASSES")) r->one_tick = strcmp(passes, "vec") == 0;
        const u64 B = s.batch, T = s.time, I = s.inputs, H = s.hidden, C = s.classes;
        r->size[0] = I * H;
        r->size[1] = H * H;
        r->size[2] = H * C;
        bool ok = hipStreamCreate(&r->stream) == hipSuccess && hipEventCreate(&r->start) == hipSuccess &&
                  hipEventCreate(&r->stop) == hipSuccess && rocblas_create_handle(&r->blas) == rocblas_status_success &&
                  rocblas_set_stream(r->blas, r->stream) == rocblas_status_success;
        for (hipEvent_t& e : r->marks)
            if (ok) ok = hipEventCreate(&e) == hipSuccess;
        auto alloc = [&](auto** p, u64 bytes) {
            if (ok) ok = hipMalloc((void**)p, bytes ? bytes : 4) == hipSuccess;
        };
        for (int k = 0; k < 3; ++k) {
            alloc(&r->w[k], r->size[k] * 4);
            alloc(&r->m[k], r->size[k] * 4);
            alloc(&r->v[k], r->size[k] * 4);
            alloc(&r->g[k], r->size[k] * 4);
        }
        alloc(&r->x, T * B * I * 4);
        alloc(&r->staging, T * B * I * 4);
        alloc(&r->hin, T * B * H * 4);
        alloc(&r->syn, B * H * 4);
        alloc(&r->mem, B * H * 4);
        alloc(&r->mem_tape, T * B * H * 4);
        alloc(&r->spikes, T * B * H * 4);
        alloc(&r->h2, T * B * C * 4);
        alloc(&r->logits, B * C * 4);
        alloc(&r->losses, B * 4);
        alloc(&r->glogit, B * C * 4);
        alloc(&r->gh2, T * B * C * 4);
        alloc(&r->gs_read, T * B * H * 4);
        alloc(&r->gmem, B * H * 4);
        alloc(&r->gsyn, B * H * 4);
        alloc(&r->g1, T * B * H * 4);
        alloc(&r->argmax, B * C * 4);
        u64 widest = I * H > H * H ? I * H : H * H;
        if (H * C > widest) widest = H * C;
        alloc(&r->partials, MAX_SPLITS * 3 * widest * 4);
        alloc(&r->x3, T * B * 3 * I * 2);
        alloc(&r->spikes16, T * B * H * 2);
        alloc(&r->g3, T * B * 3 * H * 2);
        alloc(&r->w3_in, 3 * I * H * 2);
        alloc(&r->exact, 4);
        alloc(&r->labels, B * 8);
        if (!ok) {
            delete r;
            return fail(err, cap, 2, "device allocation failed");
        }
        const float* init[3] = {w_in, w_rec, w_out};
        for (int k = 0; k < 3 && ok; ++k) {
            ok = hipMemcpy(r->w[k], init[k], r->size[k] * 4, hipMemcpyHostToDevice) == hipSuccess;
            hipLaunchKernelGGL(fill, dim3(blocks(r->size[k])), dim3(256), 0, r->stream, r->m[k], r->size[k], 0.0f);
            hipLaunchKernelGGL(fill, dim3(blocks(r->size[k])), dim3(256), 0, r->stream, r->v[k], r->size[k], 0.0f);
        }
        hipLaunchKernelGGL(split_rows, dim3(blocks(I * H)), dim3(256), 0, r->stream, I * H, r->w[0], r->w3_in);
        if (!ok || hipStreamSynchronize(r->stream) != hipSuccess) {
            delete r;
            return fail(err, cap, 3, "weight upload failed");
        }
        *out = r;
        return 0;
    } catch (...) {
        return fail(err, cap, 7, "host exception");
    }
}

void atlas_rsnn_destroy(AtlasRsnn* r) { delete r; }

int atlas_rsnn_set_batch(AtlasRsnn* r, const float* x, const uint64_t* labels, char* err, size_t cap) {
    if (!r || !x || !labels) return fail(err, cap, 7, "null argument");
    const AtlasRsnnSpec& s = r->spec;
    const u64 n = s.batch * s.time * s.inputs;
    for (u64 b = 0; b < s.batch; ++b)
        if (labels[b] >= s.classes) return fail(err, cap, 7, "label out of range");
    if (hipSetDevice(r->device) != hipSuccess) return fail(err, cap, 1, "hipSetDevice failed");
    if (hipMemcpyAsync(r->staging, x, n * 4, hipMemcpyHostToDevice, r->stream) != hipSuccess ||
        hipMemcpyAsync(r->labels, labels, s.batch * 8, hipMemcpyHostToDevice, r->stream) != hipSuccess)
        return fail(err, cap, 3, "batch upload failed");
    hipLaunchKernelGGL(fill_int, dim3(1), dim3(1), 0, r->stream, r->exact, 1);
    hipLaunchKernelGGL(to_tick_major, dim3(blocks(n)), dim3(256), 0, r->stream, s.batch, s.time, s.inputs, r->staging,
                       r->x, r->x3, r->exact);
    int exact = 0;
    if (hipStreamSynchronize(r->stream) != hipSuccess ||
        hipMemcpy(&exact, r->exact, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
        return fail(err, cap, 4, "batch transpose failed");
    r->binary_inputs = exact != 0;
    r->has_batch = true;
    return 0;
}

int atlas_rsnn_step(AtlasRsnn* r, int train, uint64_t repeats, float* losses, float* logits, double* device_ms,
                    char* err, size_t cap) {
    try {
        if (!r || !r->has_batch) return fail(err, cap, 7, "no batch set");
        if (hipSetDevice(r->device) != hipSuccess) return fail(err, cap, 1, "hipSetDevice failed");
        if (hipEventRecord(r->start, r->stream) != hipSuccess) return fail(err, cap, 1, "event record failed");
        for (uint64_t k = 0; k < (repeats ? repeats : 1); ++k)
            if (int rc = run_step(r, train != 0, err, cap)) return rc;
        if (hipEventRecord(r->stop, r->stream) != hipSuccess) return fail(err, cap, 1, "event record failed");
        const hipError_t sync = hipStreamSynchronize(r->stream);
        if (sync != hipSuccess) return fail(err, cap, 4, "step failed: %s", hipGetErrorString(sync));
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, r->start, r->stop);
        r->last_ms = ms;
        if (device_ms) *device_ms = ms;
        const AtlasRsnnSpec& s = r->spec;
        if (losses && hipMemcpy(losses, r->losses, s.batch * 4, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(err, cap, 5, "readback failed");
        if (logits && hipMemcpy(logits, r->logits, s.batch * s.classes * 4, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(err, cap, 5, "readback failed");
        return 0;
    } catch (...) {
        return fail(err, cap, 7, "host exception");
    }
}

int atlas_rsnn_profile(AtlasRsnn* r, int train, double* phase_ms, char* err, size_t cap) {
    try {
        if (!r || !r->has_batch || !phase_ms) return fail(err, cap, 7, "no batch set or null argument");
        if (hipSetDevice(r->device) != hipSuccess) return fail(err, cap, 1, "hipSetDevice failed");
        r->profiling = true;
        const int rc = run_step(r, train != 0, err, cap);
        r->profiling = false;
        if (rc) return rc;
        const hipError_t sync = hipStreamSynchronize(r->stream);
        if (sync != hipSuccess) return fail(err, cap, 4, "step failed: %s", hipGetErrorString(sync));
        const int phases = train ? ATLAS_RSNN_PHASES : 3;
        for (int k = 0; k < ATLAS_RSNN_PHASES; ++k) {
            float ms = 0.0f;
            if (k < phases && hipEventElapsedTime(&ms, r->marks[k], r->marks[k + 1]) != hipSuccess)
                return fail(err, cap, 1, "event timing failed");
            phase_ms[k] = k < phases ? ms : 0.0;
        }
        return 0;
    } catch (...) {
        return fail(err, cap, 7, "host exception");
    }
}

int atlas_rsnn_read(AtlasRsnn* r, uint32_t what, float* host, uint64_t count, char* err, size_t cap) {
    if (!r || !host) return fail(err, cap, 7, "null argument");
    const AtlasRsnnSpec& s = r->spec;
    const u64 TBH = s.time * s.batch * s.hidden;
    const float* src = nullptr;
    u64 n = 0;
    switch (what) {
        case 0: case 1: case 2: src = r->w[what]; n = r->size[what]; break;
        case 3: case 4: case 5: src = r->g[what - 3]; n = r->size[what - 3]; break;
        case 6: src = r->spikes; n = TBH; break;
        case 7: src = r->mem_tape; n = TBH; break;
        default: return fail(err, cap, 7, "unknown buffer %u", what);
    }
    if (count != n) return fail(err, cap, 7, "buffer holds %llu values", (unsigned long long)n);
    if (hipSetDevice(r->device) != hipSuccess || hipMemcpy(host, src, n * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(err, cap, 5, "readback failed");
    return 0;
}

}  // extern "C"
