// libatlas_train_hip.so: native LIF surrogate-gradient training on one MI355X.
//
// b2_train_hip_v2 (exported also as b2_train_cuda_v2 for drop-in use by the
// reference host, gpu.rs:153-172 / training_cuda.cu:92-101) runs the dense
// layered LIF plan of the v2 metadata ABI (gpu.rs:286-341): forward over T ticks,
// mean-spike readout, cross-entropy, and the fast-sigmoid surrogate BPTT with
// optional TBPTT cuts, returning per-sample gradients that the host sums in f64
// and feeds to its f64 optimizer.  Semantics follow the reference kernel
// (training_metal.metal:46-114): every float32 sum keeps the reference's order,
// so the result equals a sequential float32 evaluation of the same loops.
//
// Parallel layout (the reference runs one sample per lane): one work-item per
// (sample, neuron) for the threshold and input-accumulation phases of a tick and
// for the two backward phases of a tick, and one work-item per (sample, weight)
// for the per-sample gradient, which sums its tick contributions in the
// reference's descending-tick order from a tape of the backward carries.
//
// Projection-graph plans (b2-lif-training-plan-v2: meta[10] = G ordered edges
// (is_input, source, target, parameter) at meta[84 + 4e], tied parameter indices;
// training_metal.metal:190-263, gpu.rs:319-341) take the same kernels with the layer
// loops replaced by edge lists: the host sorts the edge ids by target, by source and
// by parameter, keeping ascending edge order within each list, so a target's inputs,
// a source's adjoint and a parameter's gradient sum in the reference's order.  Their
// pre tape has two planes, u and the membrane after the tick's edges (before the zero
// reset), as the reference returns it.
//
// Exponential and logarithm of the readout are the shared f64 implementations
// rounded to float32 (atlas_math.h), identical on the CPU oracle.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <mutex>
#include <vector>

#include "device/atlas_math.h"
#include "../../include/atlas_train.h"

namespace {

typedef uint64_t u64;
typedef uint32_t u32;

constexpr int MAX_LAYERS = 23;  // sizes live in meta[16 .. 39]

struct Net {
    u64 B, T, L, I, N, E, C;
    u32 reset_zero, detach, window, backward;
    u32 size[MAX_LAYERS + 1];   // size[0] = inputs, size[l + 1] = neurons of layer l
    u32 noff[MAX_LAYERS + 1];   // first neuron of layer l
    u64 woff[MAX_LAYERS + 1];   // first weight of layer l (source-major: w[i * size[l+1] + j])
    float beta[MAX_LAYERS], theta[MAX_LAYERS];
    float slope, sscale, lscale;
    u64 G;   // projection-graph edges (0: dense layered plan)
};

// Edge lists of a projection graph, device resident: edge e is (input, source, target,
// parameter) at rec[4e]; in/out/par are CSR lists of edge ids by target, by (non-input)
// source and by parameter, ascending within each list.
struct Graph {
    const u32* rec;
    const u32 *in_ptr, *in_list, *out_ptr, *out_list, *par_ptr, *par_list;
};

__device__ __forceinline__ u32 layer_of(const Net& n, u32 k) {
    u32 l = 0;
    while (l + 1 < n.L && k >= n.noff[l + 1]) ++l;
    return l;
}

// ------------------------------------------------------------------ forward
__global__ void init_state(Net n, const float* __restrict__ initial, float* __restrict__ membrane,
                           float* __restrict__ carry) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    membrane[x] = initial[x];
    carry[x] = 0.0f;
}

// u = beta V; s = u > theta; V = u (reset to zero) or u - theta s (subtraction).
__global__ void forward_threshold(Net n, u64 t, float* __restrict__ membrane, float* __restrict__ pre,
                                  float* __restrict__ spike) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    const u64 b = x / n.N, k = x % n.N;
    const u32 l = layer_of(n, (u32)k);
    const float u = n.beta[l] * membrane[x];
    const float s = (u > n.theta[l]) ? 1.0f : 0.0f;
    const u64 at = (b * n.T + t) * n.N + k;
    pre[at] = u;
    spike[at] = s;
    membrane[x] = n.reset_zero ? u : u - n.theta[l] * s;
}

// V += sum_i w[i][j] * input_i in ascending i, inputs = x(t) for layer 0 and the
// previous layer's spikes of this tick otherwise; then the zero reset.  The
// value before the reset is kept for the backward pass.
__global__ void forward_input(Net n, u64 t, const float* __restrict__ xin, const float* __restrict__ w,
                              float* __restrict__ membrane, const float* __restrict__ spike,
                              float* __restrict__ before_reset) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    const u64 b = x / n.N, k = x % n.N;
    const u32 l = layer_of(n, (u32)k);
    const u32 j = (u32)k - n.noff[l], fan_in = n.size[l], fan_out = n.size[l + 1];
    const float* wl = w + n.woff[l] + j;
    const u64 at = (b * n.T + t) * n.N;
    const float* input = l ? spike + at + n.noff[l - 1] : xin + (b * n.T + t) * n.I;
    float v = membrane[x];
    for (u32 i = 0; i < fan_in; ++i) v = v + wl[(u64)i * fan_out] * input[i];
    before_reset[at + k] = v;
    membrane[x] = n.reset_zero ? v * (1.0f - spike[at + k]) : v;
}

// Projection graph: V += w[param] * input over the edges into this neuron in ascending
// edge order (inputs: x(t) for input edges, this tick's spikes otherwise), the value kept
// as the second pre plane, then the zero reset.
__global__ void graph_forward_input(Net n, Graph g, u64 t, const float* __restrict__ xin, const float* __restrict__ w,
                                    float* __restrict__ membrane, const float* __restrict__ spike,
                                    float* __restrict__ before_reset) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    const u64 b = x / n.N, k = x % n.N;
    const u64 at = (b * n.T + t) * n.N;
    const float* xt = xin + (b * n.T + t) * n.I;
    float v = membrane[x];
    for (u32 q = g.in_ptr[k]; q < g.in_ptr[k + 1]; ++q) {
        const u32* e = g.rec + 4 * (u64)g.in_list[q];
        const float input = e[0] ? xt[e[1]] : spike[at + e[1]];
        v = v + w[e[3]] * input;
    }
    before_reset[at + k] = v;
    membrane[x] = n.reset_zero ? v * (1.0f - spike[at + k]) : v;
}

// logits = sum_t spike * scale / T (ascending t); loss = max + log(sum exp(logit - max)) - logit[label].
__global__ void readout(Net n, const float* __restrict__ spike, const u64* __restrict__ labels,
                        float* __restrict__ logits, float* __restrict__ losses, float* __restrict__ norm) {
    const u64 b = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n.B) return;
    const u32 out = n.noff[n.L - 1];
    float maxlog = -__builtin_huge_valf();
    for (u64 j = 0; j < n.C; ++j) {
        float sum = 0.0f;
        for (u64 t = 0; t < n.T; ++t) sum = sum + spike[(b * n.T + t) * n.N + out + j] * n.lscale / (float)n.T;
        logits[b * n.C + j] = sum;
        maxlog = fmaxf(maxlog, sum);
    }
    float denom = 0.0f;
    for (u64 j = 0; j < n.C; ++j) denom = denom + atlas_expf(logits[b * n.C + j] - maxlog);
    losses[b] = maxlog + atlas_logf(denom) - logits[b * n.C + labels[b]];
    norm[2 * b] = maxlog;
    norm[2 * b + 1] = denom;
}

// ----------------------------------------------------------------- backward
// g(t) = carry * (1 - s(t)) (zero reset) or carry: the gradient reaching the
// input accumulation of tick t.
__device__ __forceinline__ float carry_gate(const Net& n, float carry, float s) {
    return n.reset_zero ? carry * (1.0f - s) : carry;
}

// ds of tick t: the readout term for output neurons; for a hidden neuron i of
// layer l, sum_j g(t)[layer l+1, j] * w[i][j] in ascending j.
__global__ void backward_ds(Net n, u64 t, const float* __restrict__ w, const float* __restrict__ gate,
                            const float* __restrict__ logits, const float* __restrict__ norm,
                            const u64* __restrict__ labels, float* __restrict__ ds) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    const u64 b = x / n.N, k = x % n.N;
    const u32 l = layer_of(n, (u32)k);
    if (l == n.L - 1) {
        const u64 j = k - n.noff[l];
        const float e = atlas_expf(logits[b * n.C + j] - norm[2 * b]);
        float d = (e / norm[2 * b + 1] - (j == labels[b] ? 1.0f : 0.0f)) / (float)n.B;
        ds[x] = d * n.lscale / (float)n.T;
        return;
    }
    const u32 i = (u32)k - n.noff[l], fan_out = n.size[l + 2];
    const float* wl = w + n.woff[l + 1] + (u64)i * fan_out;
    const float* g = gate + (b * n.T + t) * n.N + n.noff[l + 1];
    float sum = 0.0f;
    for (u32 j = 0; j < fan_out; ++j) sum = sum + g[j] * wl[j];
    ds[x] = sum;
}

// Projection graph: ds of tick t is the readout term (output neurons) plus, over the
// neuron's out-edges in ascending edge order, g(t)[target] * w[param].
__global__ void graph_backward_ds(Net n, Graph g, u64 t, const float* __restrict__ w, const float* __restrict__ gate,
                                  const float* __restrict__ logits, const float* __restrict__ norm,
                                  const u64* __restrict__ labels, float* __restrict__ ds) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    const u64 b = x / n.N, k = x % n.N;
    const u32 out = n.noff[n.L - 1];
    float sum = 0.0f;
    if (k >= out) {
        const u64 j = k - out;
        const float e = atlas_expf(logits[b * n.C + j] - norm[2 * b]);
        const float d = (e / norm[2 * b + 1] - (j == labels[b] ? 1.0f : 0.0f)) / (float)n.B;
        sum = d * n.lscale / (float)n.T;
    }
    const float* gt = gate + (b * n.T + t) * n.N;
    for (u32 q = g.out_ptr[k]; q < g.out_ptr[k + 1]; ++q) {
        const u32* e = g.rec + 4 * (u64)g.out_list[q];
        sum = sum + gt[e[2]] * w[e[3]];
    }
    ds[x] = sum;
}

// carry(t-1) = beta (carry * dV/du + ds * phi), phi = scale / (1 + slope |u - theta|)^2,
// zeroed at TBPTT boundaries; then the gate g(t-1) for the next backward tick.
__global__ void backward_carry(Net n, u64 t, const float* __restrict__ pre, const float* __restrict__ spike,
                               const float* __restrict__ before_reset, const float* __restrict__ ds,
                               float* __restrict__ carry, float* __restrict__ gate) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.N) return;
    const u64 b = x / n.N, k = x % n.N;
    const u32 l = layer_of(n, (u32)k);
    const u64 at = (b * n.T + t) * n.N + k;
    const float u = pre[at], s = spike[at];
    const float q = 1.0f + n.slope * fabsf(u - n.theta[l]);
    const float phi = n.sscale / (q * q);
    const float derivative = n.reset_zero ? (1.0f - s - (n.detach ? 0.0f : before_reset[at] * phi))
                                          : (1.0f - (n.detach ? 0.0f : n.theta[l] * phi));
    const float previous = n.beta[l] * (carry[x] * derivative + ds[x] * phi);
    const float next = (t > 0 && t % n.window == 0) ? 0.0f : previous;
    carry[x] = next;
    if (t > 0) gate[at - n.N] = carry_gate(n, next, spike[at - n.N]);
}

// Per-sample gradient of weight e = (i, j) of layer l: sum over descending t of
// g(t)[j] * input_i(t).
__global__ void backward_grad(Net n, const float* __restrict__ xin, const float* __restrict__ spike,
                              const float* __restrict__ gate, float* __restrict__ grad) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.E) return;
    const u64 b = x / n.E, e = x % n.E;
    u32 l = 0;
    while (l + 1 < n.L && e >= n.woff[l + 1]) ++l;
    const u64 local = e - n.woff[l];
    const u32 fan_out = n.size[l + 1];
    const u32 i = (u32)(local / fan_out), j = (u32)(local % fan_out);
    const u32 k = n.noff[l] + j;
    float acc = 0.0f;
    for (u64 t = n.T; t-- > 0;) {
        const u64 at = (b * n.T + t) * n.N;
        const float input = l ? spike[at + n.noff[l - 1] + i] : xin[(b * n.T + t) * n.I + i];
        acc = acc + gate[at + k] * input;
    }
    grad[x] = acc;
}

// Projection graph: per-sample gradient of parameter p, over descending t and, within a
// tick, its edges in ascending order, of g(t)[target] * input(t).
__global__ void graph_backward_grad(Net n, Graph g, const float* __restrict__ xin, const float* __restrict__ spike,
                                    const float* __restrict__ gate, float* __restrict__ grad) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n.B * n.E) return;
    const u64 b = x / n.E, p = x % n.E;
    float acc = 0.0f;
    for (u64 t = n.T; t-- > 0;) {
        const u64 at = (b * n.T + t) * n.N;
        const float* xt = xin + (b * n.T + t) * n.I;
        for (u32 q = g.par_ptr[p]; q < g.par_ptr[p + 1]; ++q) {
            const u32* e = g.rec + 4 * (u64)g.par_list[q];
            const float input = e[0] ? xt[e[1]] : spike[at + e[1]];
            acc = acc + gate[at + e[2]] * input;
        }
    }
    grad[x] = acc;
}

// Zero-fill of a float buffer: the clears of the gate and gradient buffers are kernels, ordered
// on the stream with the kernels that use them.
__global__ void fill_zero(float* p, u64 n) {
    const u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// Device workspace of b2_train_hip_v2_static: every per-call device buffer (the staged
// inputs, the outputs before read-back, the tapes) is carved out of this array instead of
// hipMalloc'd.  Each GPU the library runs on holds its own copy until the process ends.
// In host code the name is not a device address: its per-device address comes from
// hipGetSymbolAddress (static_scratch below).
constexpr size_t STATIC_SCRATCH_BYTES = size_t(64) << 20;
constexpr size_t STATIC_ALIGN = 256;
static __device__ __align__(256) unsigned char scratch[STATIC_SCRATCH_BYTES];

// ------------------------------------------------------------------ host
int fail(char* err, size_t cap, int code, const char* fmt, ...) {
    if (err && cap) {
        va_list args;
        va_start(args, fmt);
        vsnprintf(err, cap, fmt, args);
        va_end(args);
    }
    return code;
}

struct Buffers {
    void* p[17] = {};
    ~Buffers() {
        for (void* v : p)
            if (v) (void)hipFree(v);
    }
};

inline unsigned grid(u64 items) { return (unsigned)((items + 255) / 256); }

int parse(const u64* m, const float* params, Net& n, char* err, size_t cap) {
    n.B = m[0]; n.T = m[1]; n.L = m[2]; n.I = m[3]; n.N = m[4]; n.E = m[5]; n.G = m[10];
    if (!n.B || !n.T || n.L < 2 || n.L > MAX_LAYERS || !n.I || !n.N)
        return fail(err, cap, 7, "invalid training metadata shape");
    for (u64 k : {(u64)11, (u64)14, (u64)15, (u64)79, (u64)80, (u64)81, (u64)82, (u64)83})
        if (m[k]) return fail(err, cap, 7,
                              "unsupported training plan (metadata word %llu set): dense layered or projection-graph "
                              "LIF only", (unsigned long long)k);
    if (m[12] < 84 + 4 * n.G || m[13] != 2 * n.L + 3)
        return fail(err, cap, 7, "unexpected metadata/parameter lengths");
    if (n.G > 0xFFFFFFFFull || n.E > 0xFFFFFFFFull) return fail(err, cap, 7, "projection graph beyond u32 indices");
    n.reset_zero = m[6] != 0;
    n.detach = m[7] != 0;
    n.window = (u32)(m[8] ? m[8] : n.T);
    n.backward = (m[9] & 1) != 0;
    u64 neurons = 0, weights = 0;
    n.size[0] = (u32)m[16];
    if (m[16] != n.I) return fail(err, cap, 7, "input size mismatch");
    for (u64 l = 0; l < n.L; ++l) {
        n.size[l + 1] = (u32)m[17 + l];
        n.noff[l] = (u32)m[40 + l];
        n.woff[l] = n.G ? 0 : m[64 + l];   // a projection graph has parameter banks, not layer weights
        if (n.noff[l] != neurons || (!n.G && n.woff[l] != weights) || !n.size[l + 1])
            return fail(err, cap, 7, "inconsistent layer offsets");
        neurons += n.size[l + 1];
        weights += (u64)n.size[l] * n.size[l + 1];
        n.beta[l] = params[l];
        n.theta[l] = params[n.L + l];
    }
    if (neurons != n.N || (!n.G && weights != n.E)) return fail(err, cap, 7, "layer sizes disagree with N/E");
    n.C = n.size[n.L];
    n.slope = params[2 * n.L];
    n.sscale = params[2 * n.L + 1];
    n.lscale = params[2 * n.L + 2];
    return 0;
}

int select_device(char* err, size_t cap) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1) return fail(err, cap, 1, "no HIP GPU");
    int device = 0;
    const char* choice = getenv("B2_TRAIN_HIP_DEVICE");
    if (!choice) choice = getenv("B2_TRAIN_CUDA_DEVICE");
    if (choice) {
        errno = 0;
        char* end = nullptr;
        const long value = strtol(choice, &end, 10);
        if (errno || end == choice || *end || value < 0 || value >= count)
            return fail(err, cap, 1, "invalid B2_TRAIN_HIP_DEVICE");
        device = (int)value;
    }
    if (hipSetDevice(device) != hipSuccess) return fail(err, cap, 1, "hipSetDevice failed");
    return 0;
}

// The device address of the current device's `scratch`, looked up once per device with that
// device current (hipGetSymbolAddress) and kept for later calls.
int static_scratch(void** base, char* err, size_t cap) {
    constexpr int MAX_DEVICES = 64;
    static std::mutex lock;
    static void* address[MAX_DEVICES] = {};
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= MAX_DEVICES)
        return fail(err, cap, 1, "no current HIP device for the static workspace");
    std::lock_guard<std::mutex> guard(lock);
    if (!address[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(err, cap, 1, "hipGetSymbolAddress of the static workspace failed: %s", hipGetErrorString(e));
        address[device] = p;
    }
    *base = address[device];
    return 0;
}

// The projection graph's edge records and its CSR lists by target, by non-input source and
// by parameter (edge ids ascending within each list), in one u32 array: rec[4G], in_ptr[N+1],
// in_list[G], out_ptr[N+1], out_list[G], par_ptr[E+1], par_list[G].  Checks every index.
int graph_lists(const u64* m, const Net& n, std::vector<u32>& data, char* err, size_t cap) {
    const u64 G = n.G, N = n.N, E = n.E;
    data.assign(4 * G + (N + 1) + G + (N + 1) + G + (E + 1) + G, 0);
    u32* rec = data.data();
    u32* in_ptr = rec + 4 * G;
    u32* in_list = in_ptr + N + 1;
    u32* out_ptr = in_list + G;
    u32* out_list = out_ptr + N + 1;
    u32* par_ptr = out_list + G;
    u32* par_list = par_ptr + E + 1;
    for (u64 e = 0; e < G; ++e) {
        const u64* q = m + 84 + 4 * e;
        if (q[0] > 1 || q[1] >= (q[0] ? n.I : N) || q[2] >= N || q[3] >= E)
            return fail(err, cap, 7, "projection graph edge %llu outside its declared domain", (unsigned long long)e);
        for (int k = 0; k < 4; ++k) rec[4 * e + k] = (u32)q[k];
        ++in_ptr[q[2] + 1];
        if (!q[0]) ++out_ptr[q[1] + 1];
        ++par_ptr[q[3] + 1];
    }
    for (u64 k = 0; k < N; ++k) {
        in_ptr[k + 1] += in_ptr[k];
        out_ptr[k + 1] += out_ptr[k];
    }
    for (u64 p = 0; p < E; ++p) par_ptr[p + 1] += par_ptr[p];
    std::vector<u32> in_at(in_ptr, in_ptr + N), out_at(out_ptr, out_ptr + N), par_at(par_ptr, par_ptr + E);
    for (u64 e = 0; e < G; ++e) {
        const u32* q = rec + 4 * e;
        in_list[in_at[q[2]]++] = (u32)e;
        if (!q[0]) out_list[out_at[q[1]]++] = (u32)e;
        par_list[par_at[q[3]]++] = (u32)e;
    }
    return 0;
}

Graph graph_view(const u32* d, const Net& n) {
    Graph g;
    g.rec = d;
    g.in_ptr = d + 4 * n.G;
    g.in_list = g.in_ptr + n.N + 1;
    g.out_ptr = g.in_list + n.G;
    g.out_list = g.out_ptr + n.N + 1;
    g.par_ptr = g.out_list + n.G;
    g.par_list = g.par_ptr + n.E + 1;
    return g;
}

// use_static: take every device buffer from the static workspace (no allocation); else
// hipMalloc them for this call and free them on return (the reference's RAII resources).
int execute(const u64* m, const float* params, const float* x, const float* w, const float* initial,
            const u64* labels, float* pre, float* spikes, float* membrane, float* gradients, float* initial_grad,
            float* logits, float* losses, char* err, size_t cap, bool use_static) {
    if (!m || !params || !x || !w || !initial || !labels || !pre || !spikes || !membrane || !gradients ||
        !initial_grad || !logits || !losses)
        return fail(err, cap, 7, "null buffer");
    Net n;
    if (int rc = parse(m, params, n, err, cap)) return rc;
    for (u64 b = 0; b < n.B; ++b)
        if (labels[b] >= n.C) return fail(err, cap, 7, "label out of range");
    if (int rc = select_device(err, cap)) return rc;
    const u64 BN = n.B * n.N, BTN = n.B * n.T * n.N;
    std::vector<u32> graph;
    if (n.G)
        if (int rc = graph_lists(m, n, graph, err, cap)) return rc;
    // inputs: x, w, initial, labels; outputs: pre (two planes for a projection graph, the
    // second the membrane before the zero reset), spike, membrane, grad, initial_grad, logits,
    // losses; scratch: carry, ds, gate, before_reset (dense plans), norm; the graph lists
    constexpr int NBUF = 17;
    const size_t sizes[NBUF] = {n.B * n.T * n.I * 4, n.E * 4, BN * 4, n.B * 8, (n.G ? 2 : 1) * BTN * 4, BTN * 4,
                                BN * 4, n.B * n.E * 4, BN * 4, n.B * n.C * 4, n.B * 4, BN * 4, BN * 4, BTN * 4,
                                n.G ? 0 : BTN * 4, n.B * 8, graph.size() * 4};
    Buffers owned;
    void* d[NBUF] = {};
    if (use_static) {
        size_t offset = 0;
        size_t at[NBUF];
        for (int k = 0; k < NBUF; ++k) {
            at[k] = offset;
            offset += (sizes[k] + STATIC_ALIGN - 1) / STATIC_ALIGN * STATIC_ALIGN;
        }
        if (offset > STATIC_SCRATCH_BYTES)
            return fail(err, cap, 2,
                        "the plan needs %zu bytes of device workspace; the static workspace holds %zu bytes", offset,
                        STATIC_SCRATCH_BYTES);
        void* base = nullptr;
        if (int rc = static_scratch(&base, err, cap)) return rc;
        for (int k = 0; k < NBUF; ++k) d[k] = static_cast<unsigned char*>(base) + at[k];
    } else {
        for (int k = 0; k < NBUF; ++k) {
            if (hipMalloc(&owned.p[k], sizes[k] ? sizes[k] : 4) != hipSuccess)
                return fail(err, cap, 2, "device allocation of %zu bytes failed", sizes[k]);
            d[k] = owned.p[k];
        }
    }
    const void* sources[4] = {x, w, initial, labels};
    for (int k = 0; k < 4; ++k)
        if (hipMemcpy(d[k], sources[k], sizes[k], hipMemcpyHostToDevice) != hipSuccess)
            return fail(err, cap, 3, "upload failed");
    if (n.G && hipMemcpy(d[16], graph.data(), sizes[16], hipMemcpyHostToDevice) != hipSuccess)
        return fail(err, cap, 3, "upload failed");
    float* dx = (float*)d[0];
    float* dw = (float*)d[1];
    float* dinit = (float*)d[2];
    u64* dlab = (u64*)d[3];
    float *dpre = (float*)d[4], *dspk = (float*)d[5], *dmem = (float*)d[6], *dgrad = (float*)d[7];
    float *digrad = (float*)d[8], *dlog = (float*)d[9], *dloss = (float*)d[10];
    float *dcarry = (float*)d[11], *dds = (float*)d[12], *dgate = (float*)d[13];
    float* dbr = n.G ? dpre + BTN : (float*)d[14];
    float* dnorm = (float*)d[15];
    const Graph dgraph = n.G ? graph_view((const u32*)d[16], n) : Graph{};
    hipLaunchKernelGGL(init_state, dim3(grid(BN)), dim3(256), 0, 0, n, dinit, dmem, dcarry);
    for (u64 t = 0; t < n.T; ++t) {
        hipLaunchKernelGGL(forward_threshold, dim3(grid(BN)), dim3(256), 0, 0, n, t, dmem, dpre, dspk);
        if (n.G)
            hipLaunchKernelGGL(graph_forward_input, dim3(grid(BN)), dim3(256), 0, 0, n, dgraph, t, dx, dw, dmem, dspk,
                               dbr);
        else
            hipLaunchKernelGGL(forward_input, dim3(grid(BN)), dim3(256), 0, 0, n, t, dx, dw, dmem, dspk, dbr);
    }
    hipLaunchKernelGGL(readout, dim3(grid(n.B)), dim3(256), 0, 0, n, dspk, dlab, dlog, dloss, dnorm);
    if (n.backward) {
        // the gate of the last tick multiplies a zero carry
        hipLaunchKernelGGL(fill_zero, dim3(grid(BTN)), dim3(256), 0, 0, dgate, BTN);
        for (u64 t = n.T; t-- > 0;) {
            if (n.G)
                hipLaunchKernelGGL(graph_backward_ds, dim3(grid(BN)), dim3(256), 0, 0, n, dgraph, t, dw, dgate, dlog,
                                   dnorm, dlab, dds);
            else
                hipLaunchKernelGGL(backward_ds, dim3(grid(BN)), dim3(256), 0, 0, n, t, dw, dgate, dlog, dnorm, dlab,
                                   dds);
            hipLaunchKernelGGL(backward_carry, dim3(grid(BN)), dim3(256), 0, 0, n, t, dpre, dspk, dbr, dds, dcarry,
                               dgate);
        }
        if (n.G)
            hipLaunchKernelGGL(graph_backward_grad, dim3(grid(n.B * n.E)), dim3(256), 0, 0, n, dgraph, dx, dspk, dgate,
                               dgrad);
        else
            hipLaunchKernelGGL(backward_grad, dim3(grid(n.B * n.E)), dim3(256), 0, 0, n, dx, dspk, dgate, dgrad);
    } else {
        hipLaunchKernelGGL(fill_zero, dim3(grid(n.B * n.E)), dim3(256), 0, 0, dgrad, n.B * n.E);
    }
    if (hipGetLastError() != hipSuccess) return fail(err, cap, 4, "kernel launch failed");
    const hipError_t sync = hipDeviceSynchronize();
    if (sync != hipSuccess) return fail(err, cap, 4, "kernel execution failed: %s", hipGetErrorString(sync));
    void* targets[7] = {pre, spikes, membrane, gradients, initial_grad, logits, losses};
    const int order[7] = {4, 5, 6, 7, 11, 9, 10};   // initial_grad is the final carry
    for (int k = 0; k < 7; ++k)
        if (hipMemcpy(targets[k], d[order[k]], sizes[order[k]], hipMemcpyDeviceToHost) != hipSuccess)
            return fail(err, cap, 5, "readback failed");
    return 0;
}

}  // namespace

extern "C" {

int b2_train_hip_v2(const uint64_t* meta, const float* params, const float* x, const float* w, const float* initial,
                    const uint64_t* labels, float* pre, float* spikes, float* membrane, float* gradients,
                    float* initial_grad, float* logits, float* losses, char* error, size_t capacity) {
    try {
        return execute(meta, params, x, w, initial, labels, pre, spikes, membrane, gradients, initial_grad, logits,
                       losses, error, capacity, false);
    } catch (const std::exception& e) {
        return fail(error, capacity, 7, "HIP host runtime: %s", e.what());
    } catch (...) {
        return fail(error, capacity, 7, "HIP host runtime failed");
    }
}

int b2_train_hip_v2_static(const uint64_t* meta, const float* params, const float* x, const float* w,
                           const float* initial, const uint64_t* labels, float* pre, float* spikes, float* membrane,
                           float* gradients, float* initial_grad, float* logits, float* losses, char* error,
                           size_t capacity) {
    try {
        return execute(meta, params, x, w, initial, labels, pre, spikes, membrane, gradients, initial_grad, logits,
                       losses, error, capacity, true);
    } catch (const std::exception& e) {
        return fail(error, capacity, 7, "HIP host runtime: %s", e.what());
    } catch (...) {
        return fail(error, capacity, 7, "HIP host runtime failed");
    }
}

int b2_train_cuda_v2(const uint64_t* meta, const float* params, const float* x, const float* w, const float* initial,
                     const uint64_t* labels, float* pre, float* spikes, float* membrane, float* gradients,
                     float* initial_grad, float* logits, float* losses, char* error, size_t capacity) {
    return b2_train_hip_v2(meta, params, x, w, initial, labels, pre, spikes, membrane, gradients, initial_grad, logits,
                           losses, error, capacity);
}

uint64_t b2_train_math_v1(void) { return 1; }

}  // extern "C"
