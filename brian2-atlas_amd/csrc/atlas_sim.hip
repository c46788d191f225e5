// libatlas_sim_hip.so: resident executor behind the C ABI declared in include/atlas_sim.h.
//
// Device memory, the HIP stream, hiprtc compilation of the generated tick module,
// the per-tick launch loop, and the model-independent device kernels (fills,
// the fixed in-degree topology builder, spike-bitmap decoding) live here.  The
// model-specific tick kernels are compiled at run time from the hand-written
// templates in device/atlas_tick.h plus statement bodies generated from AtlasIR.
#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <rocprim/device/device_radix_sort.hpp>

#include "../../include/atlas_sim.h"

typedef unsigned int u32;
typedef unsigned long long u64;

struct AtlasSim {
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void*> buffers;
    std::vector<u64> sizes;
    u64* table = nullptr;          // device copy of the buffer address table
    size_t table_len = 0;
    bool table_dirty = true;
    hipModule_t module = nullptr;
    std::vector<hipFunction_t> kernels;
    std::vector<AtlasLaunch> schedule;
    std::vector<AtlasLaunch> epilogue;   // launched once after the last tick, with that tick
    // persistent mode: one cooperative launch of `persistent.kernel` runs up to persistent_ticks ticks
    AtlasLaunch persistent{};
    int64_t persistent_ticks = 0;
    uint32_t persistent_barrier = 0;   // buffer zeroed before each persistent launch
    bool persistent_plain = false;     // ordinary launches (residency checked by occupancy) instead of cooperative
    bool profiling = false;
    std::vector<double> kernel_ms;
    std::vector<u64> kernel_launches;
};

namespace {

int fail(char* err, size_t cap, int code, const char* fmt, ...) {
    if (err && cap) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, cap, fmt, ap);
        va_end(ap);
    }
    return code;
}

#define HIP_TRY(call, code)                                                                   \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return fail(err, cap, code, "%s: %s (%s:%d)", #call, hipGetErrorString(e_),       \
                        __FILE__, __LINE__);                                                  \
    } while (0)

// ------------------------------------------------------------------ fills
__global__ void fill_zero_kernel(unsigned char* p, u64 n) {
    u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    u64 stride = (u64)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = 0;
}

__global__ void fill_zero_words(u32* p, u64 n) {
    u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    u64 stride = (u64)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = 0;
}

int zero_range(AtlasSim* sim, void* base, u64 bytes, char* err, size_t cap) {
    if (!bytes) return ATLAS_OK;
    unsigned char* p = static_cast<unsigned char*>(base);
    u64 head = (4 - ((uintptr_t)p & 3)) & 3;
    if (head > bytes) head = bytes;
    if (head) {
        hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(64), 0, sim->stream, p, head);
        p += head;
        bytes -= head;
    }
    u64 words = bytes / 4;
    if (words) {
        u64 blocks = std::min<u64>((words + 255) / 256, 65536);
        hipLaunchKernelGGL(fill_zero_words, dim3((u32)blocks), dim3(256), 0, sim->stream,
                           reinterpret_cast<u32*>(p), words);
    }
    u64 tail = bytes - words * 4;
    if (tail)
        hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(64), 0, sim->stream, p + words * 4, tail);
    HIP_TRY(hipGetLastError(), ATLAS_E_KERNEL);
    return ATLAS_OK;
}

// ------------------------------------------------ fixed in-degree topology
// mix64 with the golden-gamma pre-add and draw()/bounded() of
// brian2-rust/src/large_topology.rs:54-71.
__device__ __forceinline__ u64 topo_mix64(u64 v) {
    v += 0x9e3779b97f4a7c15ULL;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
    return v ^ (v >> 31);
}
__device__ __forceinline__ u64 topo_bounded(u64 seed, u64 stream, u64 edge, u64 upper) {
    u64 d = topo_mix64(seed ^ (stream * 0xd2b74407b1ce6e93ULL) ^ (edge * 0x9e3779b97f4a7c15ULL));
    return __umul64hi(d, upper);
}

__device__ __forceinline__ u32 hash_slot(u32 key, u32 log2cap) {
    return (key * 2654435761u) >> (32 - log2cap);
}

// Floyd's subset sampling per target (large_topology.rs:189-211), one wavefront
// per target.  The 64 lanes draw 64 consecutive candidates at once; membership
// in the already-selected set is an LDS hash lookup, and the dependencies
// inside a batch (a draw equal to an earlier lane's selection) are resolved in
// lane order, so the result equals the sequential algorithm.
__global__ void __launch_bounds__(256) floyd_kernel(u64 n_src, u64 k_in, u64 seed, u64 n_tgt,
                                                     u32 log2cap, u32 waves, u32 target_start,
                                                     u32* __restrict__ keys,
                                                     u32* __restrict__ values) {
    extern __shared__ u32 table_lds[];
    const u32 wave = threadIdx.x >> 6;
    const u32 lane = threadIdx.x & 63;
    const u32 capn = 1u << log2cap;
    u32* h = table_lds + (u64)wave * capn;
    const u64 first = n_src - k_in;
    for (u64 t = (u64)blockIdx.x * waves + wave; t < n_tgt; t += (u64)gridDim.x * waves) {
        for (u32 q = lane; q < capn; q += 64) h[q] = 0;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        for (u64 c0 = first; c0 < n_src; c0 += 64) {
            const u64 c = c0 + lane;
            const bool active = c < n_src;
            u32 draw = 0;
            bool collided = false;
            if (active) {
                draw = (u32)topo_bounded(seed, 0, t * n_src + c, c + 1);
                u32 slot = hash_slot(draw, log2cap);
                for (;;) {
                    u32 v = h[slot];
                    if (v == 0) break;
                    if (v == draw + 1) { collided = true; break; }
                    slot = (slot + 1) & (capn - 1);
                }
            }
            const u32 limit = (u32)min<u64>(64, n_src - c0);
            for (u32 j = 0; j < limit; ++j) {
                const u32 mine = collided ? (u32)c : draw;
                const u32 sel_j = __shfl(mine, (int)j, 64);
                if (lane > j && active && !collided && draw == sel_j) collided = true;
            }
            const u32 sel = collided ? (u32)c : draw;
            if (active) {
                u32 slot = hash_slot(sel, log2cap);
                while (atomicCAS(&h[slot], 0u, sel + 1) != 0u) slot = (slot + 1) & (capn - 1);
                const u64 pos = t * k_in + (c - first);
                keys[pos] = sel;
                values[pos] = (u32)(t + target_start);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// The rows of one source must list its targets strictly ascending: the pairs were generated
// target-major and the radix sort is stable, so row r is then the reference's source-major edge
// id r (build_fixed_indegree_indices, large_topology.rs:232-261), on which per-edge procedural
// parameters are drawn.  Any other order sets *bad.
__global__ void row_order_check(const u32* __restrict__ sorted_keys, const u32* __restrict__ row_target, u64 n,
                                u32* __restrict__ bad) {
    for (u64 r = (u64)blockIdx.x * blockDim.x + threadIdx.x; r + 1 < n; r += (u64)gridDim.x * blockDim.x)
        if (sorted_keys[r] == sorted_keys[r + 1] && row_target[r] >= row_target[r + 1]) *bad = 1u;
}

// First row position of each source in the source-sorted key array.
__global__ void row_offsets_kernel(const u32* __restrict__ sorted_keys, u64 n, u64 n_src,
                                   u64* __restrict__ offsets) {
    u64 s = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (s > n_src) return;
    u64 lo = 0, hi = n;
    while (lo < hi) {
        u64 m = (lo + hi) >> 1;
        if (sorted_keys[m] < s) lo = m + 1; else hi = m;
    }
    offsets[s] = lo;
}

// segment[s * (blocks + 1) + b] = first row position of source s whose target
// lies in block b or later.
__global__ void segment_kernel(const u32* __restrict__ row_target, const u64* __restrict__ offsets,
                               u64 n_src, u64 blocks, u64 block, u32* __restrict__ segment) {
    u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    const u64 per = blocks + 1;
    if (i >= n_src * per) return;
    const u64 s = i / per, b = i % per;
    u64 lo = offsets[s], hi = offsets[s + 1];
    const u64 bound = b * block;
    while (lo < hi) {
        u64 m = (lo + hi) >> 1;
        if ((u64)row_target[m] < bound) lo = m + 1; else hi = m;
    }
    segment[i] = (u32)lo;
}

// Slot table of a counting delivery.  Segment x = (g, b) of the segment table (g the
// (source, delay group) row, b the target block; b == blocks is the row's end
// marker) gets the slot y = xcd * groups * per_xcd + g * per_xcd + w % per_xcd with
// w = first_block + b the block's workgroup index and xcd = w / per_xcd the die its
// workgroup runs on: each XCD's slots form one contiguous region, so the random
// per-source reads of one die stay within 1/xcds of the table (TLB reach), and a
// source's slots for the die's consecutive blocks share cache lines.  A slot (two
// uint4, 16 u16 words) holds the segment's count in word 0 and, for at most 15
// targets, the targets as block-local indices in words 1..15; a longer segment keeps
// its first row in u32 word 1 instead, and its targets are read from the row table.
// *max_count collects the largest count (a table with a count above 65535 does not
// fit the count word and must not be used); *bad is set when a segment lies outside
// the row table.
// With row_slots (the edge-keyed lists of ordered groups) every slot keeps its first row in u32
// word 1, and only a segment of at most 12 targets has them inline, in u16 words 4..15.
__global__ void slot_kernel(const u32* __restrict__ segment, const u32* __restrict__ row_target, u64 rows,
                            u64 groups, u64 blocks, u64 block, u64 first_block, u64 per_xcd, u32 row_slots,
                            uint4* __restrict__ slots, u32* __restrict__ max_count, u32* __restrict__ bad) {
    const u64 x = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= groups * (blocks + 1)) return;
    const u64 g = x / (blocks + 1), b = x % (blocks + 1);
    if (b == blocks) return;
    const u32 lo = segment[x], hi = segment[x + 1];
    if (lo > hi || hi > rows) {
        *bad = 1u;
        return;
    }
    u32 w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    const u32 n = hi - lo;
    atomicMax(max_count, n);
    w[0] = n & 0xFFFFu;
    if (row_slots) {
        w[1] = lo;
        if (n <= 12u)
            for (u32 r = 0; r < n; ++r) {
                const u32 local = row_target[lo + r] - (u32)(b * block);
                const u32 k = r + 4;
                w[k / 2] |= (local & 0xFFFFu) << (16u * (k % 2));
            }
    } else if (n > 15u) {
        w[1] = lo;
    } else {
        for (u32 r = 0; r < n; ++r) {
            const u32 local = row_target[lo + r] - (u32)(b * block);
            const u32 k = r + 1;
            w[k / 2] |= (local & 0xFFFFu) << (16u * (k % 2));
        }
    }
    const u64 wg = first_block + b;
    const u64 y = (wg / per_xcd) * groups * per_xcd + g * per_xcd + wg % per_xcd;
    slots[2 * y] = make_uint4(w[0], w[1], w[2], w[3]);
    slots[2 * y + 1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// --------------------------------------------------------- spike decoding
__global__ void bitmap_row_counts(const u32* __restrict__ bits, u64 rows, u64 words,
                                  u32* __restrict__ counts) {
    __shared__ u32 partial[256];
    const u64 row = blockIdx.x;
    if (row >= rows) return;
    u32 c = 0;
    for (u64 w = threadIdx.x; w < words; w += 256) c += __popc(bits[row * words + w]);
    partial[threadIdx.x] = c;
    __syncthreads();
    for (u32 s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) partial[threadIdx.x] += partial[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[row] = partial[0];
}

__global__ void bitmap_row_pairs(const u32* __restrict__ bits, u64 rows, u64 words, u64 neurons,
                                 const u64* __restrict__ row_start, long long* __restrict__ pairs) {
    __shared__ u32 scan[257];
    const u64 row = blockIdx.x;
    if (row >= rows) return;
    u64 base = row_start[row];
    for (u64 w0 = 0; w0 < words; w0 += 256) {
        const u64 w = w0 + threadIdx.x;
        const u32 word = w < words ? bits[row * words + w] : 0u;
        scan[threadIdx.x + 1] = __popc(word);
        if (threadIdx.x == 0) scan[0] = 0;
        __syncthreads();
        if (threadIdx.x == 0)
            for (u32 k = 1; k <= 256; ++k) scan[k] += scan[k - 1];
        __syncthreads();
        u64 out = base + scan[threadIdx.x];
        u32 bitsleft = word;
        while (bitsleft) {
            const u32 b = __ffs(bitsleft) - 1;
            bitsleft &= bitsleft - 1;
            const u64 neuron = w * 32 + b;
            if (neuron < neurons) {
                pairs[2 * out] = (long long)row;
                pairs[2 * out + 1] = (long long)neuron;
            }
            ++out;
        }
        base += scan[256];
        __syncthreads();
    }
}

int upload_table(AtlasSim* sim, char* err, size_t cap) {
    if (!sim->table_dirty) return ATLAS_OK;
    if (sim->table) HIP_TRY(hipFree(sim->table), ATLAS_E_ALLOC);
    sim->table = nullptr;
    sim->table_len = sim->buffers.size();
    std::vector<u64> host(sim->table_len + 1, 0);
    for (size_t k = 0; k < sim->table_len; ++k) host[k] = reinterpret_cast<u64>(sim->buffers[k]);
    HIP_TRY(hipMalloc(&sim->table, host.size() * sizeof(u64)), ATLAS_E_ALLOC);
    HIP_TRY(hipMemcpy(sim->table, host.data(), host.size() * sizeof(u64), hipMemcpyHostToDevice),
            ATLAS_E_UPLOAD);
    sim->table_dirty = false;
    return ATLAS_OK;
}

}  // namespace

extern "C" {

int atlas_sim_create(int device, AtlasSim** out, char* err, size_t cap) {
    if (!out) return fail(err, cap, ATLAS_E_HOST, "null output handle");
    *out = nullptr;
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count), ATLAS_E_DEVICE);
    if (device < 0 || device >= count)
        return fail(err, cap, ATLAS_E_DEVICE, "device %d out of range (%d devices)", device, count);
    HIP_TRY(hipSetDevice(device), ATLAS_E_DEVICE);
    AtlasSim* sim = new (std::nothrow) AtlasSim();
    if (!sim) return fail(err, cap, ATLAS_E_HOST, "out of host memory");
    sim->device = device;
    hipError_t e = hipStreamCreateWithFlags(&sim->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete sim;
        return fail(err, cap, ATLAS_E_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    *out = sim;
    return ATLAS_OK;
}

int atlas_sim_device_name(AtlasSim* sim, char* name, size_t name_cap, char* err, size_t cap) {
    if (!sim || !name || name_cap == 0) return fail(err, cap, ATLAS_E_HOST, "null handle or name buffer");
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, sim->device), ATLAS_E_DEVICE);
    snprintf(name, name_cap, "%s (%s)", prop.name, prop.gcnArchName);
    return ATLAS_OK;
}

void atlas_sim_destroy(AtlasSim* sim) {
    if (!sim) return;
    (void)hipSetDevice(sim->device);
    (void)hipStreamSynchronize(sim->stream);
    if (sim->module) (void)hipModuleUnload(sim->module);
    for (void* p : sim->buffers)
        if (p) (void)hipFree(p);
    if (sim->table) (void)hipFree(sim->table);
    (void)hipStreamDestroy(sim->stream);
    delete sim;
}

int atlas_sim_alloc(AtlasSim* sim, uint64_t bytes, const void* host_init, uint32_t* buffer, char* err,
                    size_t cap) {
    if (!sim || !buffer) return fail(err, cap, ATLAS_E_HOST, "null argument");
    HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
    void* p = nullptr;
    const u64 padded = bytes ? (bytes + 255) / 256 * 256 : 256;
    HIP_TRY(hipMalloc(&p, padded), ATLAS_E_ALLOC);
    sim->buffers.push_back(p);
    sim->sizes.push_back(bytes);
    sim->table_dirty = true;
    *buffer = (u32)(sim->buffers.size() - 1);
    if (host_init && bytes) {
        HIP_TRY(hipMemcpyAsync(p, host_init, bytes, hipMemcpyHostToDevice, sim->stream), ATLAS_E_UPLOAD);
        HIP_TRY(hipStreamSynchronize(sim->stream), ATLAS_E_UPLOAD);
    } else {
        int rc = zero_range(sim, p, padded, err, cap);
        if (rc) return rc;
        HIP_TRY(hipStreamSynchronize(sim->stream), ATLAS_E_KERNEL);
    }
    return ATLAS_OK;
}

int atlas_sim_upload(AtlasSim* sim, uint32_t buffer, uint64_t offset, const void* host, uint64_t bytes,
                     char* err, size_t cap) {
    if (!sim || buffer >= sim->buffers.size() || offset + bytes > sim->sizes[buffer])
        return fail(err, cap, ATLAS_E_HOST, "upload outside buffer %u", buffer);
    HIP_TRY(hipMemcpyAsync(static_cast<char*>(sim->buffers[buffer]) + offset, host, bytes,
                           hipMemcpyHostToDevice, sim->stream), ATLAS_E_UPLOAD);
    HIP_TRY(hipStreamSynchronize(sim->stream), ATLAS_E_UPLOAD);
    return ATLAS_OK;
}

int atlas_sim_read(AtlasSim* sim, uint32_t buffer, uint64_t offset, void* host, uint64_t bytes, char* err,
                   size_t cap) {
    if (!sim || buffer >= sim->buffers.size() || offset + bytes > sim->sizes[buffer])
        return fail(err, cap, ATLAS_E_HOST, "read outside buffer %u", buffer);
    HIP_TRY(hipStreamSynchronize(sim->stream), ATLAS_E_KERNEL);
    HIP_TRY(hipMemcpy(host, static_cast<char*>(sim->buffers[buffer]) + offset, bytes, hipMemcpyDeviceToHost),
            ATLAS_E_READBACK);
    return ATLAS_OK;
}

int atlas_sim_copy(AtlasSim* sim, uint32_t dst, uint64_t dst_offset, uint32_t src, uint64_t src_offset,
                   uint64_t bytes, char* err, size_t cap) {
    if (!sim || dst >= sim->buffers.size() || src >= sim->buffers.size() || dst_offset + bytes > sim->sizes[dst] ||
        src_offset + bytes > sim->sizes[src])
        return fail(err, cap, ATLAS_E_HOST, "copy outside buffers %u <- %u", dst, src);
    if (!bytes) return ATLAS_OK;
    HIP_TRY(hipMemcpyAsync(static_cast<char*>(sim->buffers[dst]) + dst_offset,
                           static_cast<const char*>(sim->buffers[src]) + src_offset, bytes,
                           hipMemcpyDeviceToDevice, sim->stream), ATLAS_E_KERNEL);
    return ATLAS_OK;
}

int atlas_sim_zero(AtlasSim* sim, uint32_t buffer, uint64_t offset, uint64_t bytes, char* err, size_t cap) {
    if (!sim || buffer >= sim->buffers.size() || offset + bytes > sim->sizes[buffer])
        return fail(err, cap, ATLAS_E_HOST, "zero outside buffer %u", buffer);
    return zero_range(sim, static_cast<char*>(sim->buffers[buffer]) + offset, bytes, err, cap);
}

int atlas_sim_compile(AtlasSim* sim, const char* source, const char* const* kernel_names,
                      uint32_t kernel_count, const char* const* options, uint32_t option_count, char* err,
                      size_t cap) {
    if (!sim || !source || (kernel_count && !kernel_names))
        return fail(err, cap, ATLAS_E_HOST, "null argument");
    HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, source, "atlas_model.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        return fail(err, cap, ATLAS_E_COMPILE, "hiprtcCreateProgram failed");
    std::vector<const char*> opts(options, options + option_count);
    hiprtcResult rc = hiprtcCompileProgram(prog, (int)opts.size(), opts.data());
    if (rc != HIPRTC_SUCCESS) {
        size_t log_size = 0;
        hiprtcGetProgramLogSize(prog, &log_size);
        std::string log(log_size + 1, '\0');
        hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return fail(err, cap, ATLAS_E_COMPILE, "hiprtc: %s\n%s", hiprtcGetErrorString(rc), log.c_str());
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    std::vector<char> code(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    if (sim->module) {
        HIP_TRY(hipModuleUnload(sim->module), ATLAS_E_COMPILE);
        sim->module = nullptr;
    }
    HIP_TRY(hipModuleLoadData(&sim->module, code.data()), ATLAS_E_COMPILE);
    sim->kernels.assign(kernel_count, nullptr);
    for (uint32_t k = 0; k < kernel_count; ++k)
        HIP_TRY(hipModuleGetFunction(&sim->kernels[k], sim->module, kernel_names[k]), ATLAS_E_COMPILE);
    sim->kernel_ms.assign(kernel_count, 0.0);
    sim->kernel_launches.assign(kernel_count, 0);
    return ATLAS_OK;
}

int atlas_sim_set_schedule(AtlasSim* sim, const AtlasLaunch* launches, uint32_t count, char* err,
                           size_t cap) {
    if (!sim || (count && !launches)) return fail(err, cap, ATLAS_E_HOST, "null argument");
    for (uint32_t k = 0; k < count; ++k) {
        if (launches[k].kernel >= sim->kernels.size())
            return fail(err, cap, ATLAS_E_HOST, "launch %u names unknown kernel %u", k, launches[k].kernel);
        if (!launches[k].grid_x || !launches[k].block_x || launches[k].block_x > 1024)
            return fail(err, cap, ATLAS_E_HOST, "launch %u has an invalid shape", k);
    }
    sim->schedule.assign(launches, launches + count);
    return ATLAS_OK;
}

int atlas_sim_set_epilogue(AtlasSim* sim, const AtlasLaunch* launches, uint32_t count, char* err, size_t cap) {
    if (!sim || (count && !launches)) return fail(err, cap, ATLAS_E_HOST, "null argument");
    for (uint32_t k = 0; k < count; ++k) {
        if (launches[k].kernel >= sim->kernels.size())
            return fail(err, cap, ATLAS_E_HOST, "epilogue launch %u names unknown kernel %u", k, launches[k].kernel);
        if (!launches[k].grid_x || !launches[k].block_x || launches[k].block_x > 1024)
            return fail(err, cap, ATLAS_E_HOST, "epilogue launch %u has an invalid shape", k);
    }
    sim->epilogue.assign(launches, launches + count);
    return ATLAS_OK;
}

int atlas_sim_set_profiling(AtlasSim* sim, int enabled, char* err, size_t cap) {
    if (!sim) return fail(err, cap, ATLAS_E_HOST, "null handle");
    sim->profiling = enabled != 0;
    return ATLAS_OK;
}

int atlas_sim_kernel_time(AtlasSim* sim, uint32_t kernel, double* total_ms, uint64_t* launches, char* err,
                          size_t cap) {
    if (!sim || kernel >= sim->kernel_ms.size()) return fail(err, cap, ATLAS_E_HOST, "unknown kernel");
    *total_ms = sim->kernel_ms[kernel];
    *launches = sim->kernel_launches[kernel];
    return ATLAS_OK;
}

int atlas_sim_set_persistent(AtlasSim* sim, const AtlasLaunch* launch, uint32_t barrier_buffer,
                             int64_t ticks_per_launch, uint32_t flags, char* err, size_t cap) {
    if (!sim) return fail(err, cap, ATLAS_E_HOST, "null argument");
    if (ticks_per_launch <= 0) {
        sim->persistent_ticks = 0;
        return ATLAS_OK;
    }
    if (!launch || launch->kernel >= sim->kernels.size() || launch->grid_x == 0 || launch->block_x == 0)
        return fail(err, cap, ATLAS_E_HOST, "invalid persistent launch");
    if (barrier_buffer >= sim->buffers.size())
        return fail(err, cap, ATLAS_E_HOST, "invalid barrier buffer %u", barrier_buffer);
    if (flags & ~ATLAS_PERSISTENT_PLAIN) return fail(err, cap, ATLAS_E_HOST, "unknown persistent flags %u", flags);
    if (flags & ATLAS_PERSISTENT_PLAIN) {
        // an ordinary launch: every workgroup must fit at once, by the occupancy the kernel's
        // resources allow on every compute unit
        HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
        int per_cu = 0, cus = 0;
        HIP_TRY(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sim->kernels[launch->kernel],
                                                                   (int)launch->block_x, launch->shared_bytes),
                ATLAS_E_DEVICE);
        HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, sim->device), ATLAS_E_DEVICE);
        if ((int64_t)per_cu * cus < (int64_t)launch->grid_x)
            return fail(err, cap, ATLAS_E_COOPERATIVE, "%u workgroups cannot all be resident (%d per CU, %d CUs)",
                        launch->grid_x, per_cu, cus);
    }
    sim->persistent_plain = (flags & ATLAS_PERSISTENT_PLAIN) != 0;
    sim->persistent = *launch;
    sim->persistent_barrier = barrier_buffer;
    sim->persistent_ticks = ticks_per_launch;
    return ATLAS_OK;
}

namespace {
// Persistent mode: cooperative launches (every workgroup resident at once, or the launch fails
// with ATLAS_E_COOPERATIVE and nothing ran), each kernel(table, first_tick, count) running up
// to persistent_ticks ticks with a grid barrier between them.
int run_persistent(AtlasSim* sim, int64_t start_tick, int64_t ticks, u64& launches, char* err, size_t cap) {
    const AtlasLaunch& l = sim->persistent;
    hipEvent_t marks[2];
    if (sim->profiling) {
        HIP_TRY(hipEventCreate(&marks[0]), ATLAS_E_DEVICE);
        HIP_TRY(hipEventCreate(&marks[1]), ATLAS_E_DEVICE);
    }
    for (int64_t tick = start_tick; tick < start_tick + ticks; tick += sim->persistent_ticks) {
        int64_t count = std::min<int64_t>(sim->persistent_ticks, start_tick + ticks - tick);
        // the grid-barrier counters start every launch at zero (a fill kernel, ordered on the stream)
        const int rc = zero_range(sim, sim->buffers[sim->persistent_barrier], sim->sizes[sim->persistent_barrier],
                                  err, cap);
        if (rc) return rc;
        void* args[] = {&sim->table, &tick, &count};
        if (sim->profiling) HIP_TRY(hipEventRecord(marks[0], sim->stream), ATLAS_E_DEVICE);
        if (sim->persistent_plain) {
            HIP_TRY(hipModuleLaunchKernel(sim->kernels[l.kernel], l.grid_x, 1, 1, l.block_x, 1, 1, l.shared_bytes,
                                          sim->stream, args, nullptr),
                    ATLAS_E_KERNEL);
        } else {
            const hipError_t e = hipModuleLaunchCooperativeKernel(sim->kernels[l.kernel], l.grid_x, 1, 1, l.block_x,
                                                                  1, 1, l.shared_bytes, sim->stream, args);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return fail(err, cap, ATLAS_E_COOPERATIVE, "cooperative launch of %u workgroups: %s", l.grid_x,
                            hipGetErrorString(e));
            }
        }
        if (sim->profiling) {
            HIP_TRY(hipEventRecord(marks[1], sim->stream), ATLAS_E_DEVICE);
            HIP_TRY(hipEventSynchronize(marks[1]), ATLAS_E_KERNEL);
            float ms = 0.f;
            HIP_TRY(hipEventElapsedTime(&ms, marks[0], marks[1]), ATLAS_E_DEVICE);
            sim->kernel_ms[l.kernel] += ms;
            sim->kernel_launches[l.kernel] += 1;
        }
        ++launches;
    }
    if (sim->profiling) {
        (void)hipEventDestroy(marks[0]);
        (void)hipEventDestroy(marks[1]);
    }
    return ATLAS_OK;
}
}  // namespace

int atlas_sim_run(AtlasSim* sim, int64_t start_tick, int64_t ticks, AtlasRunStats* stats, char* err,
                  size_t cap) {
    if (!sim || ticks < 0) return fail(err, cap, ATLAS_E_HOST, "invalid run arguments");
    HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
    int rc = upload_table(sim, err, cap);
    if (rc) return rc;
    if (sim->persistent_ticks > 0) {
        auto host0 = std::chrono::steady_clock::now();
        hipEvent_t begin, end;
        HIP_TRY(hipEventCreate(&begin), ATLAS_E_DEVICE);
        HIP_TRY(hipEventCreate(&end), ATLAS_E_DEVICE);
        if (sim->profiling) {
            std::fill(sim->kernel_ms.begin(), sim->kernel_ms.end(), 0.0);
            std::fill(sim->kernel_launches.begin(), sim->kernel_launches.end(), 0);
        }
        HIP_TRY(hipEventRecord(begin, sim->stream), ATLAS_E_DEVICE);
        u64 launches = 0;
        rc = run_persistent(sim, start_tick, ticks, launches, err, cap);
        HIP_TRY(hipEventRecord(end, sim->stream), ATLAS_E_DEVICE);
        HIP_TRY(hipEventSynchronize(end), ATLAS_E_KERNEL);
        float device_ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&device_ms, begin, end), ATLAS_E_DEVICE);
        (void)hipEventDestroy(begin);
        (void)hipEventDestroy(end);
        if (rc) return rc;
        HIP_TRY(hipGetLastError(), ATLAS_E_KERNEL);
        if (stats) {
            stats->device_seconds = device_ms * 1e-3;
            stats->host_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - host0).count();
            stats->ticks = ticks;
            stats->launches = launches;
        }
        return ATLAS_OK;
    }
    auto host0 = std::chrono::steady_clock::now();
    hipEvent_t begin, end;
    HIP_TRY(hipEventCreate(&begin), ATLAS_E_DEVICE);
    HIP_TRY(hipEventCreate(&end), ATLAS_E_DEVICE);
    std::vector<hipEvent_t> marks;
    if (sim->profiling) {
        marks.resize(2 * std::max(sim->schedule.size(), sim->epilogue.size()) * (size_t)std::min<int64_t>(ticks, 1));
        for (auto& m : marks) HIP_TRY(hipEventCreate(&m), ATLAS_E_DEVICE);
        std::fill(sim->kernel_ms.begin(), sim->kernel_ms.end(), 0.0);
        std::fill(sim->kernel_launches.begin(), sim->kernel_launches.end(), 0);
    }
    HIP_TRY(hipEventRecord(begin, sim->stream), ATLAS_E_DEVICE);
    u64 launches = 0;
    // every tick runs the schedule; after the last tick the epilogue runs with that tick
    const int64_t last = start_tick + ticks - 1;
    const int64_t end_tick = start_tick + ticks + ((sim->epilogue.empty() || ticks == 0) ? 0 : 1);
    for (int64_t tick = start_tick; tick < end_tick; ++tick) {
        const bool tail = tick == start_tick + ticks;
        const std::vector<AtlasLaunch>& list = tail ? sim->epilogue : sim->schedule;
        int64_t arg = tail ? last : tick;
        for (size_t k = 0; k < list.size(); ++k) {
            const AtlasLaunch& l = list[k];
            void* args[] = {&sim->table, &arg};
            if (sim->profiling) HIP_TRY(hipEventRecord(marks[2 * k], sim->stream), ATLAS_E_DEVICE);
            HIP_TRY(hipModuleLaunchKernel(sim->kernels[l.kernel], l.grid_x, 1, 1, l.block_x, 1, 1,
                                          l.shared_bytes, sim->stream, args, nullptr),
                    ATLAS_E_KERNEL);
            if (sim->profiling) {
                HIP_TRY(hipEventRecord(marks[2 * k + 1], sim->stream), ATLAS_E_DEVICE);
                HIP_TRY(hipEventSynchronize(marks[2 * k + 1]), ATLAS_E_KERNEL);
                float ms = 0.f;
                HIP_TRY(hipEventElapsedTime(&ms, marks[2 * k], marks[2 * k + 1]), ATLAS_E_DEVICE);
                sim->kernel_ms[l.kernel] += ms;
                sim->kernel_launches[l.kernel] += 1;
            }
            ++launches;
        }
    }
    HIP_TRY(hipEventRecord(end, sim->stream), ATLAS_E_DEVICE);
    HIP_TRY(hipEventSynchronize(end), ATLAS_E_KERNEL);
    float device_ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&device_ms, begin, end), ATLAS_E_DEVICE);
    (void)hipEventDestroy(begin);
    (void)hipEventDestroy(end);
    for (auto& m : marks) (void)hipEventDestroy(m);
    HIP_TRY(hipGetLastError(), ATLAS_E_KERNEL);
    if (stats) {
        stats->device_seconds = device_ms * 1e-3;
        stats->host_seconds =
            std::chrono::duration<double>(std::chrono::steady_clock::now() - host0).count();
        stats->ticks = ticks;
        stats->launches = launches;
    }
    return ATLAS_OK;
}

int atlas_sim_fixed_indegree(AtlasSim* sim, const AtlasFixedIndegree* spec, char* err, size_t cap) {
    if (!sim || !spec) return fail(err, cap, ATLAS_E_HOST, "null argument");
    const u64 n_src = spec->source_count, n_tgt = spec->target_count, k_in = spec->indegree;
    const u64 edges = n_tgt * k_in;
    if (!n_src || !n_tgt || !k_in || k_in > n_src || edges > 0xFFFFFFFFULL || n_src > 0xFFFFFFFFULL ||
        spec->target_start + n_tgt > 0xFFFFFFFFULL)
        return fail(err, cap, ATLAS_E_HOST, "invalid fixed-indegree topology specification");
    if (spec->row_target_buffer >= sim->buffers.size() || spec->segment_buffer >= sim->buffers.size() ||
        sim->sizes[spec->row_target_buffer] < edges * 4 ||
        sim->sizes[spec->segment_buffer] < n_src * (spec->blocks + 1) * 4)
        return fail(err, cap, ATLAS_E_HOST, "fixed-indegree output buffers too small");
    if (spec->block == 0 || spec->blocks * spec->block < spec->target_start + n_tgt)
        return fail(err, cap, ATLAS_E_HOST, "target blocks do not cover the projection");
    HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
    u32 log2cap = 7;
    while ((1ull << log2cap) < 2 * k_in) ++log2cap;
    if (log2cap > 14) return fail(err, cap, ATLAS_E_HOST, "indegree %llu exceeds the LDS hash capacity",
                                  (unsigned long long)k_in);
    const u32 waves = std::max<u32>(1, std::min<u32>(4, (u32)(16384u >> log2cap)));
    u32 *keys = nullptr, *values = nullptr, *keys_sorted = nullptr, *bad = nullptr;
    u64* offsets = nullptr;
    void* temp = nullptr;
    auto release = [&]() {
        if (bad) (void)hipFree(bad);
        if (keys) (void)hipFree(keys);
        if (values) (void)hipFree(values);
        if (keys_sorted) (void)hipFree(keys_sorted);
        if (offsets) (void)hipFree(offsets);
        if (temp) (void)hipFree(temp);
    };
#define BUILD_TRY(call, code)                                                                  \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) {                                                                \
            release();                                                                         \
            return fail(err, cap, code, "%s: %s", #call, hipGetErrorString(e_));               \
        }                                                                                      \
    } while (0)
    BUILD_TRY(hipMalloc(&keys, edges * 4), ATLAS_E_ALLOC);
    BUILD_TRY(hipMalloc(&values, edges * 4), ATLAS_E_ALLOC);
    BUILD_TRY(hipMalloc(&keys_sorted, edges * 4), ATLAS_E_ALLOC);
    BUILD_TRY(hipMalloc(&offsets, (n_src + 1) * 8), ATLAS_E_ALLOC);
    const u64 grid = std::min<u64>((n_tgt + waves - 1) / waves, 65536);
    hipLaunchKernelGGL(floyd_kernel, dim3((u32)grid), dim3(64 * waves), (size_t)waves * (4u << log2cap),
                       sim->stream, n_src, k_in, spec->seed, n_tgt, log2cap, waves,
                       (u32)spec->target_start, keys, values);
    BUILD_TRY(hipGetLastError(), ATLAS_E_KERNEL);
    u32 end_bit = 1;
    while (end_bit < 32 && (1ull << end_bit) < n_src) ++end_bit;
    u32* row_target = static_cast<u32*>(sim->buffers[spec->row_target_buffer]);
    size_t temp_bytes = 0;
    BUILD_TRY(rocprim::radix_sort_pairs(nullptr, temp_bytes, keys, keys_sorted, values, row_target,
                                        (size_t)edges, 0, end_bit, sim->stream), ATLAS_E_KERNEL);
    BUILD_TRY(hipMalloc(&temp, temp_bytes ? temp_bytes : 1), ATLAS_E_ALLOC);
    BUILD_TRY(rocprim::radix_sort_pairs(temp, temp_bytes, keys, keys_sorted, values, row_target,
                                        (size_t)edges, 0, end_bit, sim->stream), ATLAS_E_KERNEL);
    BUILD_TRY(hipMalloc(&bad, 4), ATLAS_E_ALLOC);
    BUILD_TRY(hipMemsetAsync(bad, 0, 4, sim->stream), ATLAS_E_KERNEL);
    hipLaunchKernelGGL(row_order_check, dim3((u32)std::min<u64>((edges + 255) / 256, 65536)), dim3(256), 0, sim->stream,
                       keys_sorted, row_target, edges, bad);
    BUILD_TRY(hipGetLastError(), ATLAS_E_KERNEL);
    hipLaunchKernelGGL(row_offsets_kernel, dim3((u32)((n_src + 256) / 256)), dim3(256), 0, sim->stream,
                       keys_sorted, edges, n_src, offsets);
    BUILD_TRY(hipGetLastError(), ATLAS_E_KERNEL);
    const u64 seg_items = n_src * (spec->blocks + 1);
    hipLaunchKernelGGL(segment_kernel, dim3((u32)((seg_items + 255) / 256)), dim3(256), 0, sim->stream,
                       row_target, offsets, n_src, spec->blocks, spec->block,
                       static_cast<u32*>(sim->buffers[spec->segment_buffer]));
    BUILD_TRY(hipGetLastError(), ATLAS_E_KERNEL);
    u32 unordered = 0;
    BUILD_TRY(hipMemcpyAsync(&unordered, bad, 4, hipMemcpyDeviceToHost, sim->stream), ATLAS_E_KERNEL);
    BUILD_TRY(hipStreamSynchronize(sim->stream), ATLAS_E_KERNEL);
    release();
#undef BUILD_TRY
    if (unordered) return fail(err, cap, ATLAS_E_KERNEL, "fixed-indegree rows are not in source-major edge order");
    return ATLAS_OK;
}

int atlas_sim_build_slots(AtlasSim* sim, const AtlasSlotTable* spec, uint32_t* max_count, char* err, size_t cap) {
    if (!sim || !spec || !max_count) return fail(err, cap, ATLAS_E_HOST, "null argument");
    if (spec->segment_buffer >= sim->buffers.size() || spec->row_target_buffer >= sim->buffers.size() ||
        spec->slot_buffer >= sim->buffers.size())
        return fail(err, cap, ATLAS_E_HOST, "unknown buffer");
    const u64 groups = spec->groups, blocks = spec->blocks, per_xcd = spec->per_xcd;
    if (!blocks || !spec->block || spec->block > 65536 || !per_xcd || !spec->xcds ||
        spec->first_block + blocks > spec->xcds * per_xcd ||
        sim->sizes[spec->segment_buffer] < groups * (blocks + 1) * 4 ||
        sim->sizes[spec->slot_buffer] < spec->xcds * groups * per_xcd * 32)
        return fail(err, cap, ATLAS_E_HOST, "slot table does not match the segment table");
    HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
    u32* flags = nullptr;
    HIP_TRY(hipMalloc(&flags, 8), ATLAS_E_ALLOC);
    hipError_t e = hipMemsetAsync(flags, 0, 8, sim->stream);
    const u64 items = groups * (blocks + 1);
    if (e == hipSuccess && items) {
        hipLaunchKernelGGL(slot_kernel, dim3((u32)((items + 255) / 256)), dim3(256), 0, sim->stream,
                           static_cast<const u32*>(sim->buffers[spec->segment_buffer]),
                           static_cast<const u32*>(sim->buffers[spec->row_target_buffer]),
                           sim->sizes[spec->row_target_buffer] / 4, groups, blocks, (u64)spec->block,
                           (u64)spec->first_block, per_xcd, spec->row_slots,
                           static_cast<uint4*>(sim->buffers[spec->slot_buffer]), flags, flags + 1);
        e = hipGetLastError();
    }
    u32 host[2] = {0u, 0u};
    if (e == hipSuccess) e = hipMemcpyAsync(host, flags, 8, hipMemcpyDeviceToHost, sim->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(sim->stream);
    (void)hipFree(flags);
    if (e != hipSuccess) return fail(err, cap, ATLAS_E_KERNEL, "slot build failed: %s", hipGetErrorString(e));
    if (host[1]) return fail(err, cap, ATLAS_E_HOST, "segment table lies outside the row table");
    *max_count = host[0];
    return ATLAS_OK;
}

int atlas_sim_extract_spikes(AtlasSim* sim, uint32_t bitmap_buffer, uint64_t rows, uint64_t words,
                             uint64_t neurons, int64_t* pairs_host, uint64_t capacity, uint64_t* count,
                             char* err, size_t cap) {
    if (!sim || bitmap_buffer >= sim->buffers.size() || sim->sizes[bitmap_buffer] < rows * words * 4 || !count)
        return fail(err, cap, ATLAS_E_HOST, "invalid spike bitmap arguments");
    HIP_TRY(hipSetDevice(sim->device), ATLAS_E_DEVICE);
    *count = 0;
    if (!rows) return ATLAS_OK;
    const u32* bits = static_cast<const u32*>(sim->buffers[bitmap_buffer]);
    u32* counts = nullptr;
    u64* starts = nullptr;
    long long* pairs = nullptr;
    HIP_TRY(hipMalloc(&counts, rows * 4), ATLAS_E_ALLOC);
    hipLaunchKernelGGL(bitmap_row_counts, dim3((u32)rows), dim3(256), 0, sim->stream, bits, rows, words, counts);
    std::vector<u32> host_counts(rows);
    hipError_t e = hipStreamSynchronize(sim->stream);
    if (e == hipSuccess) e = hipMemcpy(host_counts.data(), counts, rows * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        (void)hipFree(counts);
        return fail(err, cap, ATLAS_E_KERNEL, "spike counts: %s", hipGetErrorString(e));
    }
    std::vector<u64> host_starts(rows);
    u64 total = 0;
    for (u64 r = 0; r < rows; ++r) {
        host_starts[r] = total;
        total += host_counts[r];
    }
    *count = total;
    if (total && pairs_host && capacity >= total) {
        e = hipMalloc(&starts, rows * 8);
        if (e == hipSuccess) e = hipMalloc(&pairs, total * 16);
        if (e == hipSuccess) e = hipMemcpy(starts, host_starts.data(), rows * 8, hipMemcpyHostToDevice);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(bitmap_row_pairs, dim3((u32)rows), dim3(256), 0, sim->stream, bits, rows, words,
                               neurons, starts, pairs);
            e = hipStreamSynchronize(sim->stream);
        }
        if (e == hipSuccess) e = hipMemcpy(pairs_host, pairs, total * 16, hipMemcpyDeviceToHost);
    }
    (void)hipFree(counts);
    if (starts) (void)hipFree(starts);
    if (pairs) (void)hipFree(pairs);
    if (e != hipSuccess) return fail(err, cap, ATLAS_E_KERNEL, "spike pairs: %s", hipGetErrorString(e));
    return ATLAS_OK;
}

}  // extern "C"
