/*
 * C ABI of the MI355X (gfx950) Brian2-Atlas simulation engine, libatlas_sim_hip.so.
 *
 * The reference has no stable native ABI for GPU simulation: its CUDA engine is
 * Python that generates kernels per plan and launches them through CuPy
 * (brian2-rust/python/brian2_rust/cuda.py:80-392, CudaExecutor; per-(stage, tick)
 * launches at cuda.py:211-218).  This library is the native layer under the
 * Python executor that replaces CudaExecutor (atlas_hip.executor.HipExecutor).
 * It is a resident executor: the host lowers an AtlasIR document into device
 * buffers, one hiprtc-compiled module of tick kernels and a per-tick launch
 * list; the library owns device memory, the HIP stream and the tick loop.
 *
 * Conventions (as training_cuda.cu:16-95 for the training ABI):
 *   - every call returns 0 on success or an ATLAS_E_* code, and writes a
 *     NUL-terminated message into (err, cap) on failure;
 *   - the caller owns host memory, the library owns device memory;
 *   - one host thread and one HIP stream per handle.
 */
#ifndef ATLAS_SIM_H
#define ATLAS_SIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ATLAS_OK = 0,
    ATLAS_E_DEVICE = 1,    /* no/invalid device, stream or event failure */
    ATLAS_E_ALLOC = 2,     /* device allocation failed */
    ATLAS_E_UPLOAD = 3,    /* host->device copy failed */
    ATLAS_E_KERNEL = 4,    /* kernel launch or execution failed */
    ATLAS_E_READBACK = 5,  /* device->host copy failed */
    ATLAS_E_COMPILE = 6,   /* hiprtc compilation or module load failed */
    ATLAS_E_HOST = 7,      /* invalid argument or host-side exception */
    ATLAS_E_COOPERATIVE = 8, /* a persistent launch's workgroups cannot all be resident; nothing ran */
};

typedef struct AtlasSim AtlasSim;

/* One kernel launch of the per-tick schedule.  Every tick kernel has the
 * signature  kernel(const uint64_t* table, int64_t tick)  where table[k] is
 * the device address of buffer k. */
typedef struct {
    uint32_t kernel;      /* index into the names passed to atlas_sim_compile */
    uint32_t grid_x;      /* workgroups */
    uint32_t block_x;     /* work-items per workgroup */
    uint32_t shared_bytes;/* dynamic LDS */
} AtlasLaunch;

typedef struct {
    double device_seconds;   /* HIP-event time of the launched ticks */
    double host_seconds;     /* wall time of atlas_sim_run */
    int64_t ticks;           /* ticks executed */
    uint64_t launches;       /* kernel launches issued */
} AtlasRunStats;

/* Fixed in-degree procedural projection (restates build_fixed_indegree_indices,
 * brian2-rust/src/large_topology.rs:189-261) built directly in device memory as
 * source-major rows: row_target[p] holds the target population index
 * (target_start + local target) of row position p, rows ascending by target,
 * which is the reference edge order; segment[s * (blocks + 1) + b] is the first
 * row position of source s whose target lies in block b (block size `block`). */
typedef struct {
    uint64_t source_count;
    uint64_t target_count;
    uint64_t indegree;
    uint64_t seed;
    uint64_t target_start;       /* offset of the projection's targets in their population */
    uint64_t block;              /* neurons per target block */
    uint64_t blocks;             /* target population blocks */
    uint32_t row_target_buffer;  /* u32[target_count * indegree] */
    uint32_t segment_buffer;     /* u32[source_count * (blocks + 1)] */
} AtlasFixedIndegree;

int atlas_sim_create(int device, AtlasSim** out, char* err, size_t cap);
void atlas_sim_destroy(AtlasSim* sim);
/* The handle's device as "<marketing name> (<gcn arch>)", NUL-terminated into (name, name_cap):
 * the `device` string of the result dictionary (the reference reports its CUDA device name,
 * cuda.py:380-391). */
int atlas_sim_device_name(AtlasSim* sim, char* name, size_t name_cap, char* err, size_t cap);

/* Allocate a device buffer of `bytes`, initialised from `host_init` (bytes long)
 * or zero-filled when host_init is NULL.  Returns its table index. */
int atlas_sim_alloc(AtlasSim* sim, uint64_t bytes, const void* host_init, uint32_t* buffer,
                    char* err, size_t cap);
int atlas_sim_upload(AtlasSim* sim, uint32_t buffer, uint64_t offset, const void* host,
                     uint64_t bytes, char* err, size_t cap);
int atlas_sim_read(AtlasSim* sim, uint32_t buffer, uint64_t offset, void* host, uint64_t bytes,
                   char* err, size_t cap);
/* Copy `bytes` from buffer src (at src_offset) to buffer dst (at dst_offset) on the device. */
int atlas_sim_copy(AtlasSim* sim, uint32_t dst, uint64_t dst_offset, uint32_t src, uint64_t src_offset,
                   uint64_t bytes, char* err, size_t cap);
/* Zero-fill a byte range of a buffer (with a fill kernel, never a memset node). */
int atlas_sim_zero(AtlasSim* sim, uint32_t buffer, uint64_t offset, uint64_t bytes, char* err,
                   size_t cap);

/* Compile a HIP source for gfx950 with hiprtc and load the named kernels. */
int atlas_sim_compile(AtlasSim* sim, const char* source, const char* const* kernel_names,
                      uint32_t kernel_count, const char* const* options, uint32_t option_count,
                      char* err, size_t cap);
/* Set the launch list executed once per tick, in order. */
int atlas_sim_set_schedule(AtlasSim* sim, const AtlasLaunch* launches, uint32_t count, char* err,
                           size_t cap);
/* Launches run once after the last tick of every atlas_sim_run (with ticks > 0), each as
 * kernel(table, last_tick): a schedule that delivers each tick's delay-0 events in the next
 * tick's launch finishes the run with them.  No counterpart in the reference (its schedule
 * steps on the host, executor.rs:3927-4361). */
int atlas_sim_set_epilogue(AtlasSim* sim, const AtlasLaunch* launches, uint32_t count, char* err,
                           size_t cap);
/* Persistent mode (ticks_per_launch > 0; 0 turns it off): atlas_sim_run then issues cooperative
 * launches of `launch` (grid, work-items, LDS), each as kernel(table, first_tick, count) running
 * `count` <= ticks_per_launch consecutive ticks, instead of the per-tick schedule; buffer
 * `barrier_buffer` (the kernel's grid-barrier words) is zero-filled before each launch.  A grid
 * whose workgroups cannot all be resident fails with ATLAS_E_COOPERATIVE before any work.
 * flags: ATLAS_PERSISTENT_PLAIN issues ordinary launches instead, once the kernel's occupancy
 * shows every workgroup fits at once (rocprofv3 kernel tracing ends the process before writing
 * its output after a cooperative launch); the kernel's waits are bounded either way.  No
 * counterpart in the reference: its persistent replays are CUDA cooperative grids of generated
 * kernels (cuda_cooperative.py:27-63). */
#define ATLAS_PERSISTENT_PLAIN 1u
int atlas_sim_set_persistent(AtlasSim* sim, const AtlasLaunch* launch, uint32_t barrier_buffer,
                             int64_t ticks_per_launch, uint32_t flags, char* err, size_t cap);
/* Execute ticks [start_tick, start_tick + ticks). */
int atlas_sim_run(AtlasSim* sim, int64_t start_tick, int64_t ticks, AtlasRunStats* stats,
                  char* err, size_t cap);

/* Device topology builder (see AtlasFixedIndegree). */
int atlas_sim_fixed_indegree(AtlasSim* sim, const AtlasFixedIndegree* spec, char* err, size_t cap);

/* Slot table of a counting delivery group, built from a pathway's segment and row
 * tables (either builder).  Segment (g, b) — g the (source, delay group) row of
 * the segment table, b < blocks the target block — gets the 32-byte slot
 * y = xcd * groups * per_xcd + g * per_xcd + w % per_xcd, w = first_block + b the
 * block's workgroup index, xcd = w / per_xcd its die (slot_buffer holds
 * xcds * groups * per_xcd slots).  A slot is 16 u16 words: the segment's event
 * count, then its first 15 targets as block-local indices (target - b * block); a
 * segment of more than 15 keeps its first row in u32 word 1 instead.  With
 * row_slots set (ordered groups, whose events are keyed by edge id) every slot
 * keeps its first row in u32 word 1, and up to 12 targets in u16 words 4..15.
 * *max_count receives the largest segment; the table is usable while it is at most
 * 65535.  No reference counterpart: the reference walks its CSR per event
 * (executor.rs:2292-2382); this is the MI355X layout that turns the segment and
 * row loads of a delivery into one 32-byte load. */
typedef struct {
    uint32_t segment_buffer;     /* u32[groups * (blocks + 1)] */
    uint32_t row_target_buffer;  /* u32 rows, population-relative targets */
    uint32_t slot_buffer;        /* uint4[2 * xcds * groups * per_xcd] */
    uint32_t block;              /* neurons per block */
    uint64_t groups;             /* sources x delay groups */
    uint64_t blocks;             /* target population blocks */
    uint64_t first_block;        /* workgroup index of the population's first block */
    uint64_t per_xcd;            /* consecutive workgroup indices per die */
    uint64_t xcds;
    uint32_t row_slots;          /* 1: first row in every slot, up to 12 inline targets */
} AtlasSlotTable;

int atlas_sim_build_slots(AtlasSim* sim, const AtlasSlotTable* spec, uint32_t* max_count, char* err,
                          size_t cap);

/* Decode a spike-recording bitmap (u32 words, `words` per tick row, `rows` rows)
 * into ascending (row, neuron) pairs: writes up to `capacity` pairs as int64
 * (row, neuron) into `pairs_host` and the total count into *count. */
int atlas_sim_extract_spikes(AtlasSim* sim, uint32_t bitmap_buffer, uint64_t rows, uint64_t words,
                             uint64_t neurons, int64_t* pairs_host, uint64_t capacity,
                             uint64_t* count, char* err, size_t cap);

/* Procedural projections materialised on the host (no device, no handle), as the reference
 * prepares them for its GPU engines (brian2_rust/gpu_initialization.py prepare_model,
 * "rust-host-f64-v0"): the engine lowers them as explicit topologies.  Outputs are caller-owned.
 *
 * Fixed in-degree (large_topology.rs:213-261, build_fixed_indegree_indices): targets x indegree
 * edges, source-major, each source's edges by target ascending; local indices. */
int atlas_prepare_fixed_indegree(uint64_t sources, uint64_t targets, uint64_t indegree, uint64_t seed,
                                 uint32_t* source_out, uint32_t* target_out, char* err, size_t cap);
/* Fixed total with replacement (large_topology.rs:147-187, build_fixed_total_indices): `edges`
 * edges, source-major, each source's edges in generation order. */
int atlas_prepare_fixed_total(uint64_t sources, uint64_t targets, uint64_t edges, uint64_t seed,
                              uint32_t* source_out, uint32_t* target_out, char* err, size_t cap);
/* Per-edge initializer values out[0..count) (large_topology.rs:87-142; executor.rs:139-188):
 * kind 0 uniform in [minimum, maximum] (materialize_uniform), kind 1 clipped normal
 * (materialize_clipped_normal: mean + std * Box-Muller draw with the host libm, redrawn until
 * within the bounds the has_* flags enable, at most 1000 attempts).  ATLAS_E_HOST with the
 * reference's message for an invalid specification or an exhausted rejection loop. */
int atlas_prepare_initializer(int kind, uint64_t count, uint64_t seed, uint64_t stream, double minimum,
                              double maximum, double mean, double std_dev, int has_minimum, int has_maximum,
                              double* out, char* err, size_t cap);

/* Milliseconds of device time of the most recent launch of `kernel` measured
 * by HIP events on the library's stream during the last atlas_sim_run with
 * profiling enabled (0 disables per-kernel events). */
int atlas_sim_set_profiling(AtlasSim* sim, int enabled, char* err, size_t cap);
int atlas_sim_kernel_time(AtlasSim* sim, uint32_t kernel, double* total_ms, uint64_t* launches,
                          char* err, size_t cap);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_SIM_H */
