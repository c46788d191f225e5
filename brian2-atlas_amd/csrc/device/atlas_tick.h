// Hand-written gfx950 building blocks of the Brian2-Atlas tick kernels.
//
// The model-specific parts (state-update / threshold / reset statement bodies and
// the per-event on_pre programs) are generated from AtlasIR and compiled together
// with this header by hiprtc.  The generated code defines, before this header:
//   ATLAS_BLOCK      neurons per workgroup block (a multiple of ATLAS_WG)
//   ATLAS_WG         work-items per workgroup (a multiple of 64, at most 1024)
//   ATLAS_HIST       entries of the per-target LDS counters: ATLAS_BLOCK, or
//                    ATLAS_BLOCK per pathway of the widest counting delivery group
//   ATLAS_CAP_BITS   log2 of the events staged in LDS per delivery flush
//   ATLAS_MAX_NB     largest source-population block count read by a delivery group
//   ATLAS_MAX_GNB    largest delay groups x source blocks of a multi-delay delivery group (>= 1)
//   ATLAS_MAX_NP     largest number of pathways in one delivery group
//   ATLAS_SPT        fired sources gathered per work-item per gather pass
//   ATLAS_POST_BYTES LDS bytes of the block's post-synaptic states kept resident
//                    between the update and the deliveries of a tick (0: none)
//   ATLAS_SYN_BYTES  LDS bytes of the per-edge values staged for an ordered flush (0: none)
//   ATLAS_TSTART     ATLAS_BLOCK + 1 when a delivery group is queued, else 1
//
// Workgroups are mapped to blocks XCD-aware: hardware dispatches workgroup i to
// XCD i mod 8, and the generated kernels remap i so that each XCD owns a
// contiguous range of blocks.  A fired source's segment offsets and row targets
// for that range are then read into one L2 once per tick instead of by all XCDs.
//
// Execution model (one workgroup = one block of one population, per tick):
//   phase A  state-monitor sample, fused refractory / state update / threshold
//            (and the reset when it commutes with the deliveries) for the block's
//            neurons, ascending spike compaction (wavefront ballots + one
//            workgroup barrier), publication into the spike ring.  States that
//            the deliveries touch stay in LDS when the tick is one kernel;
//   phase B  delivery of every pathway targeting this population into the
//            block's targets, write-back of the LDS-resident states, then the
//            reset of the block's fired neurons when it was not fused.
// Phase B reads spike-ring slots of earlier ticks (delay >= 1) or, for delay-0
// pathways, a slot written by the separate phase-A kernel of the same tick.
//
// Delivery order is the reference order (executor.rs:2292-2382): pathways in
// schedule order and, inside a pathway, events by emission tick ascending, then
// source ascending, then edge ascending.  A delivery group gathers the events of
// one or more non-interacting pathways that share their source and target
// populations into LDS (each pathway's events appended in its canonical order),
// buckets them by target with integer LDS atomics, sorts each bucket by the key
// (pathway, append position), and one lane applies the bucket sequentially.
// Counting groups skip the buckets: when every program of the group reads only
// the post-synaptic states it writes and per-tick constants (no per-edge data,
// no pre-synaptic state), all events of a pathway into one target apply the
// same function, so any order gives the canonical result and the group only
// counts events per (pathway, target) before applying each program that many
// times.  There are no floating-point atomics.

typedef unsigned int u32;
typedef unsigned long long u64;
typedef long long i64;
typedef unsigned short u16;
typedef unsigned char byte_t;

#define ATLAS_WAVES (ATLAS_WG / 64)
#define ATLAS_ROUNDS (ATLAS_BLOCK / ATLAS_WG)
#define ATLAS_CAP (1u << ATLAS_CAP_BITS)
#define ATLAS_PASS (ATLAS_WG * ATLAS_SPT)
#define ATLAS_BATCH 8   // independent edges per work-item whose memory operations are issued together

// Fault bits reported through the fault word (the host raises on any set bit).
#define ATLAS_FAULT_NONFINITE 1u
#define ATLAS_FAULT_TIMESTEP 2u
#define ATLAS_FAULT_REFRACTORY 4u
#define ATLAS_FAULT_QUEUE 8u   // a delivery queue overflowed (the host enlarges it and reruns)
#define ATLAS_FAULT_RANDOM 16u  // an invalid binomial probability, or a sampler's draw budget ran out
#define ATLAS_FAULT_EDGES 64u   // a persistent launch's edge-keyed lists ran out of nodes (the host replays
                                // the run with one launch per tick)

namespace atlas {

// Device buffers are global memory: the address-space-qualified pointer lets every
// access compile to global_load/store instead of flat, whose wait counters also
// track LDS and make the compiler wait for memory before LDS work.
template <class T>
using gptr = __attribute__((address_space(1))) T*;

template <class T>
__device__ __forceinline__ gptr<T> buf(const u64* __restrict__ tab, int k) {
    return (gptr<T>)(tab[k]);
}

// A load whose address is uniform and whose memory no launch writes, through the constant
// address space: a scalar load, counted apart from the vector loads, so waiting for its value
// does not wait for every vector load issued after it.
template <class T>
__device__ __forceinline__ T uniform_load(gptr<const T> p) {
    return *(const __attribute__((address_space(4))) T*)(p);
}

// Field at byte `offset` of record `row` (records of `stride` bytes) in buffer k.
template <class T>
__device__ __forceinline__ gptr<T> field(const u64* __restrict__ tab, int k, u32 row, u32 stride, u32 offset) {
    return (gptr<T>)(buf<byte_t>(tab, k) + ((u64)row * stride + offset));
}

// ring slots whose previous counts a persistent launch keeps (a ring of 2 d + 2 ticks, d <= 20)
#define ATLAS_RING_PREV 64u

struct Lds {
    u32 scan[ATLAS_WAVES + 1];
    u32 ring_prev[ATLAS_RING_PREV];   // persistent launches: the block's count in each ring slot
    u32 round_counts[ATLAS_ROUNDS * ATLAS_WAVES];
    u32 delivered[ATLAS_MAX_NP];
    u32 dense[ATLAS_PASS];
    u32 gstart[ATLAS_MAX_GNB];   // entry starts of the (delay group, source block) table
    u32 ev_row[ATLAS_CAP];
    u16 ev_tgt[ATLAS_CAP];
    u16 ev_key[ATLAS_CAP];
    u16 ev_d[ATLAS_CAP];        // delay of each staged event (queued groups)
    u16 order[ATLAS_CAP];
    u32 hist[ATLAS_HIST];
    u32 cursor[ATLAS_BLOCK];
    u32 tstart[ATLAS_TSTART];   // per-target starts of a sorted queue (queued groups)
    u64 ev_sort[ATLAS_TSTART > 1 ? ATLAS_CAP : 1];   // bucketed sort keys of queued events
    alignas(16) byte_t post[ATLAS_POST_BYTES > 0 ? ATLAS_POST_BYTES : 16];
    alignas(16) byte_t syn[ATLAS_SYN_BYTES > 0 ? ATLAS_SYN_BYTES : 16];   // staged per-edge values
};

// Workgroup barrier ordering LDS only.  Inside the tick every thread touches global
// memory of its own neurons, targets and edges only (the same thread-to-neuron map
// in every phase), so the phases' barriers exchange LDS data alone; a full
// __syncthreads() would also wait for every outstanding global load and store (the
// state loads issued before the event counting, the state stores before the spike
// publication).  Cross-thread global dependencies (phase A's spike list before an
// on_post delivery, a monitor's reads before the stores) keep full barriers.
// The value of the other lane of the pair (2i, 2i + 1) (a DPP quad permutation 1, 0, 3, 2); every
// lane of the wave must be active.
__device__ __forceinline__ u32 lane_swap(u32 x) {
    return (u32)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, true);
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Exclusive workgroup scan of one u32 per thread.  All threads must call it.
__device__ __forceinline__ u32 wg_scan(u32 v, u32& total, Lds& s) {
    const u32 lane = __lane_id();
    const u32 wave = threadIdx.x >> 6;
    u32 x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        u32 y = __shfl_up(x, off, 64);
        if (lane >= (u32)off) x += y;
    }
    if (lane == 63) s.scan[wave] = x;
    lds_barrier();
    if (threadIdx.x == 0) {
        u32 acc = 0;
        for (int w = 0; w < ATLAS_WAVES; ++w) {
            u32 t = s.scan[w];
            s.scan[w] = acc;
            acc += t;
        }
        s.scan[ATLAS_WAVES] = acc;
    }
    lds_barrier();
    u32 r = s.scan[wave] + x - v;
    total = s.scan[ATLAS_WAVES];
    lds_barrier();
    return r;
}

// Brian2 timestep() (model.rs:981-992): truncating tick conversion of an f64 time.
__device__ __forceinline__ u64 brian_timestep(double time, double dt, u32& fault) {
    double steps = (time + 1e-3 * dt) / dt;
    if (!(time >= 0.0 && steps < 9223372036854775808.0)) {
        fault |= ATLAS_FAULT_TIMESTEP;
        return 0;
    }
    return (u64)steps;
}

// First tick after a spike at `tick` (time t = tick * dt_clock) whose fixed-
// refractory recompute (executor.rs:4045-4058) yields not_refractory = true:
// the smallest c > tick with timestep(c * dt_clock - t, dt) >= period.  The
// recompute is monotone in c, so a neuron is available at tick c iff c >= until.
__device__ __forceinline__ i64 refractory_until(i64 tick, double t, double dt_clock, double dt, u64 period,
                                                u32& fault) {
    i64 c = tick + (i64)period;
    if (c <= tick) c = tick + 1;
    for (int k = 0; k < 8 && c - 1 > tick && brian_timestep((double)(c - 1) * dt_clock - t, dt, fault) >= period; ++k)
        --c;
    for (int k = 0; k < 8 && brian_timestep((double)c * dt_clock - t, dt, fault) < period; ++k) ++c;
    if (brian_timestep((double)c * dt_clock - t, dt, fault) < period ||
        (c - 1 > tick && brian_timestep((double)(c - 1) * dt_clock - t, dt, fault) >= period))
        fault |= ATLAS_FAULT_REFRACTORY;
    return c;
}

__device__ __forceinline__ void finite(double x, u32& fault) {
    if (!__builtin_isfinite(x)) fault |= ATLAS_FAULT_NONFINITE;
}

__device__ __forceinline__ void report(const u64* __restrict__ tab, int fault_buf, u32 fault) {
    if (fault) atomicOr(buf<u32>(tab, fault_buf), fault);
}

// ---------------------------------------------------------------- persistent launches
// A persistent launch runs many ticks without a kernel boundary between them.  The spike ring
// is then the only memory one workgroup reads from another inside a launch, and it crosses
// XCDs, whose L2 caches are not coherent with each other.  Instead of L2 write-back /
// invalidate fences (a whole-L2 operation per workgroup per tick, which serialises on each
// XCD's L2) or a grid barrier, every ring word carries the tick it belongs to: the upper 12
// bits of each 32-bit word hold the tick's stamp, the lower 20 bits the value (a neuron index
// or a count, so populations stay below 2^20 neurons).  Producers store words with the sc1
// (device scope) bit and never wait; a reader loads with sc1 and re-reads, after a short
// sleep, every word whose stamp is not yet its tick's.  Each word validates itself, so no
// store order is needed.  Stamps run over 1 .. 4095 (never 0, the value of a cleared word).
// A stamp alone does not make a word fresh: a slot's id words past the counts of its later
// ticks would keep an old tick's stamp for any number of ring cycles, and that stamp recurs
// every lcm(R, 4095) ticks (4095 for a ring of 3).  So each publication into a slot also
// clears the words the slot's previous tick (tick - R) wrote past its own count: after any
// publication a slot's words below its count carry its stamp and all words past it are zero.
// A reader of tick e, past the barrier of e, sees each word either as the publication of e
// left it or as that of e - R did (whose stores every producer waited for before arriving at
// barrier e - R + 1 <= e): stamp(e), stamp(e - R) or zero, and stamp(e - R) != stamp(e) for
// any ring of 1 <= R < 4095 ticks.  So a word carrying stamp(e) is the one tick e wrote.
#define ATLAS_FAULT_STALL 32u          // a ring wait ran out of polls (the launch went on)
#define ATLAS_SPIN_LIMIT (1u << 20)    // polls of one ring word, at least 0.1 s, before giving up
#define ATLAS_RING_VALUE 0xFFFFFu      // value bits of a stamped ring word
#define ATLAS_LIST_FETCH 0xFFFFFFFEu   // LDS list entry whose id is still to be read from the ring

typedef unsigned int atlas_v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32 ring_stamp(i64 tick) { return (u32)((u64)(tick + 1) % 4095u) + 1u; }
__device__ __forceinline__ u32 ring_word(u32 stamp, u32 value) { return stamp << 20 | value; }
__device__ __forceinline__ bool ring_fresh(u32 word, u32 stamp) { return (word >> 20) == stamp; }

// A persistent launch's ring record of a source block and tick: 8 stamped words, the count of
// the block's fired neurons then the first ATLAS_REC_IDS of their ids.  (64-byte records with
// 15 ids measured slower, with 2048- and with 4096-neuron blocks: the wider loads and record
// checks cost more than the rarer id fetches saved.)
#define ATLAS_REC_WORDS 8u
#define ATLAS_REC_IDS 7u

// The two 16-byte halves of a 32-byte ring record, loaded together, waited for together.
__device__ __forceinline__ void ring_load_record(const void* p, uint4* q) {
    atlas_v4u x, y;
    asm volatile("global_load_dwordx4 %0, %2, off sc1\n\t"
                 "global_load_dwordx4 %1, %2, off offset:16 sc1\n\t"
                 "s_waitcnt vmcnt(0)"
                 : "=&v"(x), "=&v"(y) : "v"(p) : "memory");
    q[0] = make_uint4(x.x, x.y, x.z, x.w);
    q[1] = make_uint4(y.x, y.y, y.z, y.w);
}

__device__ __forceinline__ u32 record_word(const uint4* q, u32 k) {
    const uint4& v = q[k / 4];
    return k % 4 == 0 ? v.x : k % 4 == 1 ? v.y : k % 4 == 2 ? v.z : v.w;
}

__device__ __forceinline__ void ring_store_u32(u32* p, u32 v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ u32 ring_load_u32(const u32* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A record is complete once its count word and the id words it uses (the first
// min(count, ATLAS_REC_IDS)) carry the tick's stamp; the words past the count are not written.
__device__ __forceinline__ bool record_fresh(const uint4* q, u32 stamp) {
    // branch-free
    const u32 n = q[0].x & ATLAS_RING_VALUE;
    u32 stale = (q[0].x >> 20) ^ stamp;
#pragma unroll
    for (u32 k = 0; k < ATLAS_REC_IDS; ++k) stale |= k < n ? (record_word(q, k + 1) >> 20) ^ stamp : 0u;
    return stale == 0;
}

// The record at p once it is complete for `stamp`; after ATLAS_SPIN_LIMIT polls the work-item
// sets ATLAS_FAULT_STALL, takes what it read and stops waiting for the rest of the launch
// (results invalid, reported by the host).
__device__ __forceinline__ void ring_wait_record(const void* p, u32 stamp, uint4* q, bool& gave_up, u32& fault) {
    ring_load_record(p, q);
    u32 spins = 0;
    while (!gave_up && !record_fresh(q, stamp)) {
        if (++spins >= ATLAS_SPIN_LIMIT) {
            gave_up = true;
            fault |= ATLAS_FAULT_STALL;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        ring_load_record(p, q);
    }
}

__device__ __forceinline__ u32 ring_wait_u32(const u32* p, u32 stamp, bool& gave_up, u32& fault) {
    u32 w = ring_load_u32(p);
    u32 spins = 0;
    while (!gave_up && !ring_fresh(w, stamp)) {
        if (++spins >= ATLAS_SPIN_LIMIT) {
            gave_up = true;
            fault |= ATLAS_FAULT_STALL;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        w = ring_load_u32(p);
    }
    return w & ATLAS_RING_VALUE;
}

// Split-phase grid barrier over the nwg workgroups of a persistent launch; barrier `it` (1, 2,
// ... within a launch; the words start at zero).  It only tells a reader when every producer
// has issued its ring stores of a tick: the stamped words then validate themselves, so the
// arrival does not wait for the stores to complete.  grid_arrive: workgroup w adds one to
// counter w mod ATLAS_BAR_GROUPS (a 64-byte line each), an atomic whose result nobody waits
// for.  grid_wait: lane g of the first wave polls counter g until it holds every arrival of
// its members: one hop from the last arrival to every waiter, where a tree of counters would
// chain two atomic round trips and a flag store.  Up to SLOTS consecutive barriers may be
// open at once: barrier it uses the counters of slot it mod SLOTS, which barrier it + SLOTS
// reuses only once barrier it is complete (the caller's waits guarantee that), so each
// slot's counters grow barrier by barrier: its m-th barrier (m = (it - 1) / SLOTS + 1) is
// complete at m arrivals per member, and a count past that still means complete.  A wait
// gives up after ATLAS_SPIN_LIMIT polls (ATLAS_FAULT_STALL; the launch goes on).  Counter g
// of slot q is the word at (q G + g) 16.
#define ATLAS_BAR_GROUPS 32u
template <u32 SLOTS>
__device__ __forceinline__ void grid_arrive(u32* bar, u32 it, u32 wg, u32 nwg) {
    constexpr u32 G = ATLAS_BAR_GROUPS;
    (void)nwg;
    // every wave has issued its ring stores; no wait for them (or for any load) to complete
    lds_barrier();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(&bar[((it % SLOTS) * G + wg % G) * 16u], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

template <u32 SLOTS>
__device__ __forceinline__ void grid_wait(const u32* bar, u32 it, u32 nwg, bool& gave_up, u32& fault) {
    constexpr u32 G = ATLAS_BAR_GROUPS;
    const u32 g = threadIdx.x;
    if (g < G && g < nwg && !gave_up) {
        const u32 target = ((it - 1u) / SLOTS + 1u) * ((nwg - g + G - 1u) / G);
        const u32* counter = &bar[((it % SLOTS) * G + g) * 16u];
        u32 spins = 0;
        while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++spins >= ATLAS_SPIN_LIMIT) {
                gave_up = true;
                fault |= ATLAS_FAULT_STALL;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    lds_barrier();   // the stamped words the workgroup reads next validate themselves
}

// ---------------------------------------------------------------- phase A
// Pop provides: N, NB, R, CNT, IDS, SMALL (the first 8 ids of every block list,
// 32 bytes per block: at ~1-2 spikes per block and tick, deliveries rarely need
// the full list), REC (recording bitmap or -1), REC_WORDS,
// WIN0 (first recorded tick), FAULT, State, record(), load(), step(), store(),
// EVENT_RINGS and publish_events(tab, tick, blk) (custom events' rings of fired
// neurons, published after the spikes by the whole workgroup).
// All loads of a work-item's neurons are issued before any arithmetic, so the
// block streams its state with one memory round trip.
// phase_a_load issues the state loads of the work-item's neurons; phase_a_run
// consumes them.  Callers may put independent work between the two (the event
// counting of counting groups), which then overlaps the loads.  The state monitor
// samples the stored states in phase_a_run, before they are overwritten.
template <class Pop>
__device__ __forceinline__ void phase_a_load(const u64* __restrict__ tab, u32 blk,
                                             typename Pop::State (&st)[ATLAS_ROUNDS]) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        const u32 j = r * ATLAS_WG + threadIdx.x;
        if (j < n) Pop::load(tab, base + j, st[r]);
    }
}

// No counted events applied inside the update (their groups apply after it).
struct NoFused {
    template <class State>
    __device__ static void apply(const u64* __restrict__, u32, u32, State&, Lds&, double, i64, u32&) {}
};

// Phase A in two parts.  phase_a_step: state-monitor sample, update and threshold
// of the block's neurons (states stay in registers), ballots and per-wave spike
// counts; it touches neither the event counters nor the spike ring, so callers may
// run it while the tick's event counting waits for memory (deliver's hook).
// phase_a_finish: Fused::apply(tab, i, j, st, s, t, tick, fault) applies the
// counted events of populations whose deliveries are all counting groups to the
// updated states in registers (same result as applying them to the stored states
// after the update, since each program reads only the states it writes, so the
// post states need no LDS residency and no second pass), then the stores, the
// recording bitmap and the publication into the spike ring.
template <class Pop>
__device__ __forceinline__ void phase_a_step(const u64* __restrict__ tab, i64 tick, double t, u32 blk,
                             typename Pop::State (&st)[ATLAS_ROUNDS], Lds& s, u64 (&masks)[ATLAS_ROUNDS],
                             u32& fault) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    Pop::record(tab, tick, base, n);
    __syncthreads();
    const u32 lane = __lane_id();
    const u32 wave = threadIdx.x >> 6;
    const int until_next = Pop::until_next(tab, tick);
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        const u32 j = r * ATLAS_WG + threadIdx.x;
        bool fired = false;
        if (j < n) fired = Pop::step(tab, base + j, t, tick, st[r], fault, until_next);
        masks[r] = __ballot(fired);
        if (lane == 0) s.round_counts[r * ATLAS_WAVES + wave] = (u32)__popcll(masks[r]);
    }
}

template <class Pop, class Fused = NoFused>
__device__ void phase_a_finish(const u64* __restrict__ tab, i64 tick, double t, u32 blk,
                               typename Pop::State (&st)[ATLAS_ROUNDS], Lds& s, const u64 (&masks)[ATLAS_ROUNDS],
                               u32 fault) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    const u32 lane = __lane_id();
    const u32 wave = threadIdx.x >> 6;
    const bool recording = Pop::REC >= 0 && tick >= Pop::WIN0;
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        const u32 j = r * ATLAS_WG + threadIdx.x;
        if (j < n) {
            Fused::apply(tab, base + j, j, st[r], s, t, tick, fault);
            Pop::store(tab, base + j, j, st[r], s.post);
        }
        if (recording && lane < 2 && r * ATLAS_WG + wave * 64 + lane * 32 < n) {
            u32* rec = buf<u32>(tab, Pop::REC) + (u64)(tick - Pop::WIN0) * Pop::REC_WORDS;
            __builtin_nontemporal_store((u32)(masks[r] >> (32 * lane)), rec + (base + r * ATLAS_WG + wave * 64) / 32 + lane);
        }
    }
    lds_barrier();
    const u32 slot = (u32)(tick % Pop::R);
    u32* ids = buf<u32>(tab, Pop::IDS) + (u64)slot * Pop::N + base;
    u32 before = 0;
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        u32 mine = before;
        for (u32 w = 0; w < ATLAS_WAVES; ++w) {
            const u32 c = s.round_counts[r * ATLAS_WAVES + w];
            if (w < wave) mine += c;
            before += c;
        }
        if ((masks[r] >> lane) & 1ull) {
            const u32 k = mine + (u32)__popcll(masks[r] & ((1ull << lane) - 1ull));
            const u32 id = base + r * ATLAS_WG + threadIdx.x;
            ids[k] = id;
            if (k < 8) buf<u32>(tab, Pop::SMALL)[((u64)slot * Pop::NB + blk) * 8 + k] = id;
        }
    }
    if (threadIdx.x == 0) buf<u32>(tab, Pop::CNT)[(u64)slot * Pop::NB + blk] = before;
    if constexpr (Pop::EVENT_RINGS) Pop::publish_events(tab, tick, blk);
    report(tab, Pop::FAULT, fault);
}

// Delay-0 plans: the previous tick's counted events (in s.hist) applied to the block's states
// in registers, before this tick's update; the same operations in the same order as
// applying them to the stored states.
template <class Pop, class Fused>
__device__ void pre_apply(const u64* __restrict__ tab, i64 tick, double t, u32 blk,
                          typename Pop::State (&st)[ATLAS_ROUNDS], Lds& s) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    u32 fault = 0;
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        const u32 j = r * ATLAS_WG + threadIdx.x;
        if (j < n) Fused::apply(tab, base + j, j, st[r], s, t, tick, fault);
    }
    report(tab, Pop::FAULT, fault);
}

template <class Pop, class Fused = NoFused>
__device__ void phase_a_run(const u64* __restrict__ tab, i64 tick, double t, u32 blk,
                            typename Pop::State (&st)[ATLAS_ROUNDS], Lds& s) {
    u64 masks[ATLAS_ROUNDS];
    u32 fault = 0;
    phase_a_step<Pop>(tab, tick, t, blk, st, s, masks, fault);
    phase_a_finish<Pop, Fused>(tab, tick, t, blk, st, s, masks, fault);
}

template <class Pop>
__device__ void phase_a(const u64* __restrict__ tab, i64 tick, double t, u32 blk, Lds& s) {
    typename Pop::State st[ATLAS_ROUNDS];
    phase_a_load<Pop>(tab, blk, st);
    phase_a_run<Pop>(tab, tick, t, blk, st, s);
}

// Write the LDS-resident post-synaptic states of the block back to memory.
template <class Pop>
__device__ void writeback(const u64* __restrict__ tab, u32 blk, Lds& s) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    for (u32 j = threadIdx.x; j < n; j += ATLAS_WG) Pop::writeback(tab, base + j, j, s.post);
}

// Several clocks: the LDS-resident post-synaptic states of a block that receives deliveries
// at a step its own clock does not advance (no update stored them there).
template <class Pop>
__device__ void stage(const u64* __restrict__ tab, u32 blk, Lds& s) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    for (u32 j = threadIdx.x; j < n; j += ATLAS_WG) Pop::stage(tab, base + j, j, s.post);
}

// ---------------------------------------------------------------- reset
template <class Pop>
__device__ void reset_phase(const u64* __restrict__ tab, i64 tick, double t, u32 blk) {
    // custom events or end-of-tick EventMonitors: the resets slot generated for the population
    if constexpr (Pop::CUSTOM) {
        Pop::custom_phase(tab, tick, t, blk);
        return;
    }
    if (Pop::RESET_FUSED) return;
    const u32 slot = (u32)(tick % Pop::R);
    const u32 count = buf<u32>(tab, Pop::CNT)[(u64)slot * Pop::NB + blk];
    const u32* ids = buf<u32>(tab, Pop::IDS) + (u64)slot * Pop::N + blk * ATLAS_BLOCK;
    u32 fault = 0;
    for (u32 k = threadIdx.x; k < count; k += ATLAS_WG) Pop::reset(tab, ids[k], t, tick, fault);
    report(tab, Pop::FAULT, fault);
}

// ---------------------------------------------------------------- PoissonInput
// Every neuron of the block runs the population's PoissonInput programs (in order) on its
// states in memory, after the tick's deliveries into the block.
template <class Pop>
__device__ void poisson_phase(const u64* __restrict__ tab, i64 tick, double t, u32 blk) {
    u32 fault = 0;
    for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) {
        const u32 i = blk * ATLAS_BLOCK + j;
        if (i < Pop::N) Pop::poisson(tab, i, t, tick, fault);
    }
    report(tab, Pop::FAULT, fault);
}

// ---------------------------------------------------------------- run_regularly
// Every neuron of the block runs the population's run_regularly programs of the tick's end (in
// schedule order) on its states in memory, after the reset.
template <class Pop>
__device__ void regular_phase(const u64* __restrict__ tab, i64 tick, double t, u32 blk) {
    u32 fault = 0;
    for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) {
        const u32 i = blk * ATLAS_BLOCK + j;
        if (i < Pop::N) Pop::regular_end(tab, i, t, tick, fault);
    }
    report(tab, Pop::FAULT, fault);
}

// ---------------------------------------------------------------- delivery
// Canonical sort key of queued staging entry k: (pathway, delay descending, row).
__device__ __forceinline__ u64 queue_key(const Lds& s, u32 k) {
    return (u64)(s.ev_key[k] >> ATLAS_CAP_BITS) << 52 | (u64)(0xFFFFu - s.ev_d[k]) << 32 | s.ev_row[k];
}

// Apply the staged events [0, nbuf) to the block's targets in canonical order.
// On entry and on exit s.hist is zero.
// With Group::PREFETCH the per-edge values the programs read are loaded for every
// staged event at once (one memory round trip, under the bucketing below) and kept in
// LDS, so each target's lane applies its events without a dependent load per event.
// With Group::SPLIT the statements that depend on the event's own edge only (synapse
// traces, weight updates: everything but the post-synaptic accumulation) run for all
// staged events at once, spread over the work-items, and each target's lane runs the
// few statements that must follow the canonical order.
// KEYED (queued groups) orders a target's events by (pathway, delay descending, row);
// otherwise by (pathway, staging position).
template <class Group, bool KEYED = Group::QUEUE>
__device__ void flush(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 nbuf, Lds& s,
                      u32& fault) {
    constexpr u32 PERE = ATLAS_CAP / ATLAS_WG;
    typename Group::Edge pre[PERE];
    if constexpr (Group::PREFETCH || Group::SPLIT) {
#pragma unroll
        for (u32 q = 0; q < PERE; ++q) {
            const u32 k = threadIdx.x + q * ATLAS_WG;
            if (k < nbuf) Group::fetch(tab, (u32)(s.ev_key[k] >> ATLAS_CAP_BITS), s.ev_row[k], pre[q]);
        }
    }
    for (u32 k = threadIdx.x; k < nbuf; k += ATLAS_WG) atomicAdd(&s.hist[s.ev_tgt[k]], 1u);
    lds_barrier();
    constexpr u32 PER = ATLAS_BLOCK / ATLAS_WG;
    u32 local = 0;
#pragma unroll
    for (u32 q = 0; q < PER; ++q) local += s.hist[threadIdx.x * PER + q];
    u32 total;
    u32 start = wg_scan(local, total, s);
#pragma unroll
    for (u32 q = 0; q < PER; ++q) {
        s.cursor[threadIdx.x * PER + q] = start;
        start += s.hist[threadIdx.x * PER + q];
    }
    lds_barrier();
    for (u32 k = threadIdx.x; k < nbuf; k += ATLAS_WG) {
        const u32 pos = atomicAdd(&s.cursor[s.ev_tgt[k]], 1u);
        s.order[pos] = s.ev_key[k];
        if constexpr (KEYED) s.ev_sort[pos] = queue_key(s, k);
    }
    if constexpr (Group::PREFETCH) {
#pragma unroll
        for (u32 q = 0; q < PERE; ++q) {
            const u32 k = threadIdx.x + q * ATLAS_WG;
            if (k < nbuf) Group::stash(pre[q], (u32)(s.ev_key[k] >> ATLAS_CAP_BITS), k, s.syn);
        }
    }
    if constexpr (Group::SPLIT) {
        // the statements of each event's own edge, for all staged events at once; the
        // values the sequential part reads go to LDS at the event's staging index
#pragma unroll
        for (u32 q = 0; q < PERE; ++q) {
            const u32 k = threadIdx.x + q * ATLAS_WG;
            if (k < nbuf)
                Group::edge_part(tab, (u32)(s.ev_key[k] >> ATLAS_CAP_BITS), s.ev_row[k], pre[q], k, s.syn, t, tick,
                                 fault);
        }
    }
    lds_barrier();
    // Canonical order inside each target's bucket, by rank: every staged event counts
    // the events of its bucket with a smaller key (keys are distinct), then moves to
    // that position.  Staged in canonical order, a key (pathway, staging position) orders
    // itself; queued events compare by (pathway, emission tick ascending = delay
    // descending, row ascending), packed into one 64-bit key.
    u32 rank[PERE];
#pragma unroll
    for (u32 q = 0; q < PERE; ++q) {
        const u32 k = threadIdx.x + q * ATLAS_WG;
        if (k >= nbuf) continue;
        const u32 j = s.ev_tgt[k];
        const u32 cnt = s.hist[j], start = s.cursor[j] - cnt;
        u32 r = 0;
        if constexpr (KEYED) {
            const u64 mine = queue_key(s, k);
            for (u32 i = start; i < start + cnt; ++i) r += s.ev_sort[i] < mine;
        } else {
            const u32 mine = s.ev_key[k];
            for (u32 i = start; i < start + cnt; ++i) r += s.order[i] < mine;
        }
        rank[q] = start + r;
    }
    lds_barrier();
#pragma unroll
    for (u32 q = 0; q < PERE; ++q) {
        const u32 k = threadIdx.x + q * ATLAS_WG;
        if (k < nbuf) s.order[rank[q]] = s.ev_key[k];
    }
    lds_barrier();
    // Each work-item owns PER targets: load their post states, apply the events in
    // order, then store, so the memory latency overlaps.
    typename Group::Post post[PER];
#pragma unroll
    for (u32 q = 0; q < PER; ++q) {
        const u32 j = threadIdx.x + q * ATLAS_WG;
        if (s.hist[j]) Group::load_post(tab, blk * ATLAS_BLOCK + j, j, post[q], s.post);
    }
#pragma unroll
    for (u32 q = 0; q < PER; ++q) {
        const u32 j = threadIdx.x + q * ATLAS_WG;
        const u32 cnt = s.hist[j];
        if (cnt) Group::apply(tab, blk * ATLAS_BLOCK + j, post[q], &s.order[s.cursor[j] - cnt], cnt, s.ev_row,
                              s.syn, t, tick, fault);
    }
#pragma unroll
    for (u32 q = 0; q < PER; ++q) {
        const u32 j = threadIdx.x + q * ATLAS_WG;
        if (s.hist[j]) Group::store_post(tab, blk * ATLAS_BLOCK + j, j, post[q], s.post);
        s.hist[j] = 0;
    }
    lds_barrier();
}

// Counting groups: s.hist[HIST_BASE + p * ATLAS_BLOCK + j] holds the events of
// pathway p into target j; each work-item applies its targets' programs that many
// times.  On exit the counters are zero.
template <class Group>
__device__ void apply_counts(const u64* __restrict__ tab, i64 tick, double t, u32 blk, Lds& s) {
    constexpr u32 PER = ATLAS_BLOCK / ATLAS_WG;
    constexpr u32 HB = Group::HIST_BASE;
    u32 fault = 0;
#pragma unroll
    for (u32 q = 0; q < PER; ++q) {
        const u32 j = threadIdx.x + q * ATLAS_WG;
        u32 any = 0;
#pragma unroll
        for (u32 p = 0; p < Group::NP; ++p) any |= s.hist[HB + p * ATLAS_BLOCK + j];
        if (any) {
            typename Group::Post post;
            Group::load_post(tab, blk * ATLAS_BLOCK + j, j, post, s.post);
            Group::apply_counts(tab, blk * ATLAS_BLOCK + j, post, &s.hist[HB + j], t, tick, fault);
            Group::store_post(tab, blk * ATLAS_BLOCK + j, j, post, s.post);
#pragma unroll
            for (u32 p = 0; p < Group::NP; ++p) s.hist[HB + p * ATLAS_BLOCK + j] = 0;
        }
    }
    report(tab, Group::FAULT, fault);
}

// Counting through the slot table (SLOTS groups): one 32-byte load per (fired source,
// pathway) gives the count of the segment (word 0) and, for up to 15 targets, its
// block-local targets (words 1..15), so counting needs no row-table round trip; a
// longer segment's targets are read from the row table (count_long_slot).  Only valid
// slots are fetched (exec-masked loads, issued back to back).
template <class Group>
__device__ __forceinline__ void load_slots(const u64* __restrict__ tab, u32 blk, const u64* at, const bool* ok,
                                           uint4* a, uint4* b) {
    constexpr u32 X = ATLAS_SPT * ATLAS_MAX_NP;
#pragma unroll
    for (u32 x = 0; x < X; ++x) {
        const u32 p = x % ATLAS_MAX_NP;
        a[x] = make_uint4(0u, 0u, 0u, 0u);
        b[x] = a[x];
        if (ok[x]) {
            const uint4* slot = Group::slot_ptr(tab, p < Group::NP ? p : 0u, at[x], blk);
            a[x] = slot[0];
            b[x] = slot[1];
        }
    }
}

// The targets of a slot whose segment is longer than its 15 inline words (word 0 the count,
// u32 word 1 the segment's first row), read from the pathway's row table and counted.
template <class Group>
__device__ __forceinline__ void count_long_slot(const u64* __restrict__ tab, u32 p, u32 n, u32 row0, u32 blk,
                                                u32* hist) {
    for (u32 r = 0; r < n; ++r) atomicAdd(&hist[Group::row_target(tab, p, row0 + r) - blk * ATLAS_BLOCK], 1u);
}

template <class Group>
__device__ __forceinline__ void count_slots(const u64* __restrict__ tab, u32 blk, const bool* ok, const uint4* a,
                                            const uint4* b, Lds& s) {
    constexpr u32 HB = Group::HIST_BASE;
    constexpr u32 X = ATLAS_SPT * ATLAS_MAX_NP;
    u32 per_path[ATLAS_MAX_NP];
#pragma unroll
    for (u32 p = 0; p < ATLAS_MAX_NP; ++p) per_path[p] = 0;
#pragma unroll
    for (u32 x = 0; x < X; ++x) {
        const u32 p = x % ATLAS_MAX_NP;
        const u32 w[8] = {a[x].x, a[x].y, a[x].z, a[x].w, b[x].x, b[x].y, b[x].z, b[x].w};
        const u32 n = ok[x] ? (w[0] & 0xFFFFu) : 0u;
        const u32 inline_n = n <= 15u ? n : 0u;
        per_path[p] += n;
        u32* hist = &s.hist[HB + (p < Group::NP ? p : 0u) * ATLAS_BLOCK];
        // the wave leaves after its longest slot (a uniform branch on the ballot), not after 15
#pragma unroll
        for (u32 r = 0; r < 15; ++r) {
            if (!__ballot(r < inline_n)) break;
            if (r < inline_n) atomicAdd(&hist[(w[(r + 1) / 2] >> (16u * ((r + 1) % 2))) & 0xFFFFu], 1u);
        }
        if (__ballot(n > 15u) && n > 15u) count_long_slot<Group>(tab, p, n, w[1], blk, hist);
    }
    // delivered-event counters: wavefront reduction, one LDS atomic per wave
#pragma unroll
    for (u32 p = 0; p < Group::NP; ++p) {
        u32 v = per_path[p];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (__lane_id() == 0 && v) atomicAdd(&s.delivered[p], v);
    }
}

// ---------------------------------------------------------------- pending events
// Events a run inherits from the run before it (a continuation): at their delivery tick
// they come before the run's own events of the same pathway, in the order given.  The
// host lays them out per (tick - PEND_START, target block) over PEND_T ticks:
// PEND_OFF[k * PEND_TB + blk] .. [+ 1] index PEND, whose entries are {row,
// block-local target | pathway << 16}.

// Counting groups: the block's pending events of the tick added to its LDS counters
// (s.hist counting region and s.delivered, both initialised; all work-items call it).
template <class Group>
__device__ void count_pending(const u64* __restrict__ tab, i64 tick, u32 blk, Lds& s) {
    const i64 k = tick - Group::PEND_START;
    if (k < 0 || k >= (i64)Group::PEND_T) return;
    const u32* off = buf<const u32>(tab, Group::PEND_OFF) + (u64)k * Group::PEND_TB + blk;
    const u32 lo = off[0], hi = off[1];
    gptr<const uint2> pend = buf<const uint2>(tab, Group::PEND);
    for (u32 e = lo + threadIdx.x; e < hi; e += ATLAS_WG) {
        const uint2 r = pend[e];
        const u32 p = r.y >> 16;
        atomicAdd(&s.hist[Group::HIST_BASE + p * ATLAS_BLOCK + (r.y & 0xFFFFu)], 1u);
        atomicAdd(&s.delivered[p], 1u);
    }
}

// Ordered groups: the block's pending events of the tick staged ATLAS_CAP at a time and
// flushed in the order given (a target's events by pathway, then position), before the
// group's own delivery of the tick.  Uniform: every work-item calls it.
template <class Group>
__device__ void deliver_pending(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 wg_index,
                                u32 wg_count, Lds& s) {
    const i64 k = tick - Group::PEND_START;
    if (k < 0 || k >= (i64)Group::PEND_T) return;
    const u32* off = buf<const u32>(tab, Group::PEND_OFF) + (u64)k * Group::PEND_TB + blk;
    const u32 lo = off[0], hi = off[1];
    if (lo == hi) return;
    gptr<const uint2> pend = buf<const uint2>(tab, Group::PEND);
    u32 fault = 0;
    lds_barrier();
    if (threadIdx.x < Group::NP) s.delivered[threadIdx.x] = 0;
    for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) s.hist[j] = 0;
    for (u32 c = lo; c < hi; c += ATLAS_CAP) {
        const u32 n = hi - c < ATLAS_CAP ? hi - c : ATLAS_CAP;
        lds_barrier();
        for (u32 e = threadIdx.x; e < n; e += ATLAS_WG) {
            const uint2 r = pend[c + e];
            const u32 p = r.y >> 16;
            s.ev_row[e] = r.x;
            s.ev_tgt[e] = (u16)(r.y & 0xFFFFu);
            s.ev_key[e] = (u16)((p << ATLAS_CAP_BITS) | e);
            atomicAdd(&s.delivered[p], 1u);
        }
        lds_barrier();
        flush<Group, false>(tab, tick, t, blk, n, s, fault);
    }
    if (threadIdx.x < Group::NP && s.delivered[threadIdx.x])
        buf<u64>(tab, Group::DELIVERED)[(u64)Group::path_index(threadIdx.x) * wg_count + wg_index] +=
            s.delivered[threadIdx.x];
    report(tab, Group::FAULT, fault);
    lds_barrier();
}

// Group provides: NP, COUNT, SRC_N, SRC_NB, SRC_R, SRC_CNT, SRC_SMALL, SRC_IDS, NG, gval(g) (distinct
// delays, descending), seg_index(id, g, blk, at[], ok[]) -> per pathway, whether
// the fired source `id` belongs to it at delay group g and the index of its
// (source, group, block) segment start; seg_ptr(tab, p); row_target(tab, p, row);
// DELIVERED, path_index(p), FAULT; Post, load_post, apply (sorting groups) or
// apply_counts (counting groups), store_post; SLOTS and slot_ptr(tab, p, at, blk)
// (counting groups whose slot tables are complete: the slot of segment `at`).
// With APPLY = false a counting group stops after counting (its counters stay in
// LDS for apply_counts, called once the block's update has run).
struct NoHook {
    __device__ void operator()() const {}
};

// hook() runs exactly once, uniformly: right after the first pass has issued its
// segment (or slot) loads, so independent work (phase_a_step) overlaps their
// latency, or at the end when no pass ran.
template <class Group, bool APPLY = true, class Hook = NoHook>
__device__ void deliver(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 wg_index, u32 wg_count,
                        i64 start_tick, Lds& s, const Hook& hook = Hook()) {
    bool hooked = false;
    const u32 base = blk * ATLAS_BLOCK;
    u32 fault = 0;
    u32 nbuf = 0;
    if (threadIdx.x < Group::NP) s.delivered[threadIdx.x] = 0;
    constexpr u32 HB = Group::HIST_BASE;
    constexpr u32 HIST = Group::COUNT ? Group::NP * ATLAS_BLOCK : ATLAS_BLOCK;
    for (u32 j = threadIdx.x; j < HIST; j += ATLAS_WG) s.hist[HB + j] = 0;
    if constexpr (Group::COUNT && Group::PEND_T > 0 && !Group::PEND_SOURCES) {
        lds_barrier();
        count_pending<Group>(tab, tick, blk, s);
    }

    // One pass over up to ATLAS_PASS fired sources: work-item w holds the consecutive
    // entries [w * SPT, w * SPT + SPT) of the pass (source id, or 0xFFFFFFFF for none,
    // and its delay group), so exclusive scans over work-items keep the canonical
    // (emission tick, source) order.  All uniform: every work-item calls it.
    auto pass = [&](const u32 (&id)[ATLAS_SPT], const u32 (&gq)[ATLAS_SPT]) {
        // Segment lookup: all addresses first (no memory access), then every load of
        // the work-item unconditionally (invalid slots read entry 0), then selects, so
        // the loads leave together instead of one round trip per branch.
        u64 at[ATLAS_SPT * ATLAS_MAX_NP];
        bool ok[ATLAS_SPT * ATLAS_MAX_NP];
#pragma unroll
        for (u32 q = 0; q < ATLAS_SPT; ++q)
            Group::seg_index(id[q], gq[q], blk, at + q * ATLAS_MAX_NP, ok + q * ATLAS_MAX_NP);
        if constexpr (Group::SLOTS) {
            constexpr u32 X = ATLAS_SPT * ATLAS_MAX_NP;
            uint4 sa[X], sb[X];
            load_slots<Group>(tab, blk, at, ok, sa, sb);
            if (!hooked) {
                hook();
                hooked = true;
            }
            count_slots<Group>(tab, blk, ok, sa, sb, s);
            return;
        }
        u32 lo[ATLAS_SPT * ATLAS_MAX_NP], hi[ATLAS_SPT * ATLAS_MAX_NP], cn[ATLAS_SPT * ATLAS_MAX_NP];
#pragma unroll
        for (u32 q = 0; q < ATLAS_SPT; ++q)
#pragma unroll
            for (u32 p = 0; p < ATLAS_MAX_NP; ++p) {
                const u32 x = q * ATLAS_MAX_NP + p;
                const u32* seg = Group::seg_ptr(tab, p < Group::NP ? p : 0u);
                const u64 a = ok[x] ? at[x] : 0ull;
                lo[x] = seg[a];
                hi[x] = seg[a + 1];
            }
        if (!hooked) {
            hook();
            hooked = true;
        }
        u32 nev = 0;
        u32 per_path[ATLAS_MAX_NP];
#pragma unroll
        for (u32 p = 0; p < ATLAS_MAX_NP; ++p) per_path[p] = 0;
#pragma unroll
        for (u32 q = 0; q < ATLAS_SPT; ++q)
#pragma unroll
            for (u32 p = 0; p < ATLAS_MAX_NP; ++p) {
                const u32 x = q * ATLAS_MAX_NP + p;
                cn[x] = ok[x] ? hi[x] - lo[x] : 0u;
                nev += cn[x];
                per_path[p] += cn[x];
            }
        // delivered-event counters: wavefront reduction, one LDS atomic per wave
#pragma unroll
        for (u32 p = 0; p < Group::NP; ++p) {
            u32 v = per_path[p];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (__lane_id() == 0 && v) atomicAdd(&s.delivered[p], v);
        }
        u32 chunk_total;
        const u32 ex = wg_scan(nev, chunk_total, s);
        // Every work-item copies its own segments: event positions ex .. ex + nev
        // of this pass, windowed into the LDS staging buffer.
        for (u32 copied = 0; copied < chunk_total;) {
            const u32 take = (chunk_total - copied < ATLAS_CAP - nbuf) ? chunk_total - copied
                                                                      : ATLAS_CAP - nbuf;
            if (ex < copied + take && ex + nev > copied) {
                u32 pos = ex;
#pragma unroll
                for (u32 q = 0; q < ATLAS_SPT * ATLAS_MAX_NP; ++q) {
                    const u32 p = q % ATLAS_MAX_NP;
                    const u32 c = cn[q];
                    if (c && pos < copied + take && pos + c > copied) {  // segment meets the window
                        const u32 r0 = pos < copied ? copied - pos : 0u;
                        const u32 r1 = pos + c > copied + take ? copied + take - pos : c;
                        for (u32 r = r0; r < r1; ++r) {
                            const u32 e = nbuf + (pos + r - copied);
                            s.ev_row[e] = lo[q] + r;
                            s.ev_key[e] = (u16)((p << ATLAS_CAP_BITS) | e);
                        }
                    }
                    pos += c;
                }
            }
            lds_barrier();
            // targets of the staged rows: up to CAP / WG independent loads per work-item
            constexpr u32 PERE = ATLAS_CAP / ATLAS_WG;
            u32 tg[PERE];
#pragma unroll
            for (u32 e = 0; e < PERE; ++e) {
                const u32 at_ = nbuf + threadIdx.x + e * ATLAS_WG;
                const bool valid = at_ < nbuf + take;
                const u32 p = valid ? (u32)(s.ev_key[at_] >> ATLAS_CAP_BITS) : 0u;
                tg[e] = Group::row_target(tab, p, valid ? s.ev_row[at_] : 0u);
            }
#pragma unroll
            for (u32 e = 0; e < PERE; ++e) {
                const u32 at_ = nbuf + threadIdx.x + e * ATLAS_WG;
                if (at_ < nbuf + take) {
                    if constexpr (Group::COUNT)
                        atomicAdd(&s.hist[HB + (u32)(s.ev_key[at_] >> ATLAS_CAP_BITS) * ATLAS_BLOCK +
                                          (tg[e] - base)], 1u);
                    else
                        s.ev_tgt[at_] = (u16)(tg[e] - base);
                }
            }
            nbuf += take;
            copied += take;
            lds_barrier();
            if (Group::COUNT || nbuf == ATLAS_CAP) {
                if constexpr (!Group::COUNT) flush<Group>(tab, tick, t, blk, nbuf, s, fault);
                nbuf = 0;
            }
        }
    };

    const u32* cnt_base = buf<const u32>(tab, Group::SRC_CNT);
    const u32* small_base = buf<const u32>(tab, Group::SRC_SMALL);
    const u32* ids_base = buf<const u32>(tab, Group::SRC_IDS);
    if constexpr (Group::PEND_SOURCES) {
        // a continuation's pending sources of this tick, through the same lookups (counting
        // group of one delay: their order is free)
        const i64 k = tick - Group::PEND_START;
        if (k >= 0 && k < (i64)Group::PEND_T) {
            const u32* off = buf<const u32>(tab, Group::PEND_OFF) + k;
            const u32 lo = off[0], n = off[1] - off[0];
            const u32* pend = buf<const u32>(tab, Group::PEND) + lo;
            for (u32 c0 = 0; c0 < n; c0 += ATLAS_PASS) {
                u32 id[ATLAS_SPT], gq[ATLAS_SPT];
#pragma unroll
                for (u32 q = 0; q < ATLAS_SPT; ++q) {
                    const u32 e = c0 + threadIdx.x * ATLAS_SPT + q;
                    id[q] = e < n ? pend[e] : 0xFFFFFFFFu;
                    gq[q] = 0u;
                }
                pass(id, gq);
            }
        }
    }
    if constexpr (Group::NG == 1) {
        const i64 emitted = tick - (i64)Group::gval(0);
        if (emitted >= start_tick) {
            const u32 slot = (u32)(emitted % Group::SRC_R);
            // Counts and cached first ids of the source population's blocks for that
            // tick, read coalesced (every workgroup reads them, so they must not be
            // scattered), then an exclusive prefix over the counts.
            const u32* cnt = cnt_base + (u64)slot * Group::SRC_NB;
            const uint4* small = reinterpret_cast<const uint4*>(small_base) + (u64)slot * Group::SRC_NB * 2;
            constexpr u32 PERB = (Group::SRC_NB + ATLAS_WG - 1) / ATLAS_WG;
            u32 mine[PERB];
            uint4 first[PERB], second[PERB];
            u32 local = 0;
#pragma unroll
            for (u32 q = 0; q < PERB; ++q) {
                const u32 k = threadIdx.x * PERB + q;
                mine[q] = k < Group::SRC_NB ? cnt[k] : 0u;
                first[q] = k < Group::SRC_NB ? small[2 * k] : make_uint4(0u, 0u, 0u, 0u);
                second[q] = k < Group::SRC_NB ? small[2 * k + 1] : make_uint4(0u, 0u, 0u, 0u);
                local += mine[q];
            }
            u32 fired_total;
            u32 acc = wg_scan(local, fired_total, s);
            u32 start[PERB];
#pragma unroll
            for (u32 q = 0; q < PERB; ++q) {
                start[q] = acc;
                acc += mine[q];
            }
            const u32* ids = ids_base + (u64)slot * Group::SRC_N;
            for (u32 c0 = 0; c0 < fired_total; c0 += ATLAS_PASS) {
                lds_barrier();
                // dense fired list of the pass: the owner of each block writes its ids
#pragma unroll
                for (u32 q = 0; q < PERB; ++q) {
                    const u32 b = threadIdx.x * PERB + q;
                    const u32 lo = start[q] > c0 ? start[q] : c0;
                    const u32 hi = start[q] + mine[q] < c0 + ATLAS_PASS ? start[q] + mine[q] : c0 + ATLAS_PASS;
                    for (u32 k = lo; k < hi; ++k) {
                        const u32 r = k - start[q];
                        s.dense[k - c0] = r == 0 ? first[q].x : r == 1 ? first[q].y : r == 2 ? first[q].z
                                        : r == 3 ? first[q].w : r == 4 ? second[q].x : r == 5 ? second[q].y
                                        : r == 6 ? second[q].z : r == 7 ? second[q].w : ids[b * ATLAS_BLOCK + r];
                    }
                }
                lds_barrier();
                u32 id[ATLAS_SPT], gq[ATLAS_SPT];
#pragma unroll
                for (u32 q = 0; q < ATLAS_SPT; ++q) {
                    const u32 k = c0 + threadIdx.x * ATLAS_SPT + q;
                    id[q] = k < fired_total ? s.dense[k - c0] : 0xFFFFFFFFu;
                    gq[q] = 0u;
                }
                pass(id, gq);
            }
        }
    } else {
        // Several delay groups: the fired sources of every group in one canonical list,
        // (group, source block, rank) with groups by descending delay, i.e. emission
        // tick ascending.  Work-item w owns the consecutive (group, block) entries
        // [w * PERC, w * PERC + PERC) of the flattened count table; one scan gives each
        // entry's start, kept in LDS, and every pass entry finds its (group, block) there
        // by binary search and loads its source id, so one gather serves all groups.
        constexpr u32 GNB = Group::NG * Group::SRC_NB;
        constexpr u32 PERC = (GNB + ATLAS_WG - 1) / ATLAS_WG;
        u32 counts[PERC];
        u32 local = 0;
#pragma unroll
        for (u32 c = 0; c < PERC; ++c) {
            const u32 e = threadIdx.x * PERC + c;
            counts[c] = 0u;
            if (e < GNB) {
                const u32 g = e / Group::SRC_NB, b = e % Group::SRC_NB;
                const i64 emitted = tick - (i64)Group::gval(g);
                if (emitted >= start_tick)
                    counts[c] = cnt_base[(u64)(emitted % Group::SRC_R) * Group::SRC_NB + b];
            }
        }
#pragma unroll
        for (u32 c = 0; c < PERC; ++c) local += counts[c];
        u32 fired_total;
        u32 acc = wg_scan(local, fired_total, s);
#pragma unroll
        for (u32 c = 0; c < PERC; ++c) {
            const u32 e = threadIdx.x * PERC + c;
            if (e < GNB) s.gstart[e] = acc;
            acc += counts[c];
        }
        lds_barrier();
        // binary-search steps over the entry starts: the work-item's SPT searches run in
        // lockstep (branch-free, fixed step count) so their LDS reads overlap
        constexpr u32 STEPS = GNB <= 1u ? 0u : 32u - __builtin_clz(GNB - 1u);
        for (u32 c0 = 0; c0 < fired_total; c0 += ATLAS_PASS) {
            u32 id[ATLAS_SPT], gq[ATLAS_SPT], found[ATLAS_SPT];
#pragma unroll
            for (u32 q = 0; q < ATLAS_SPT; ++q) found[q] = 0u;
            // found[q]: the last entry starting at or before k (empty entries share their
            // start), as the sum of the powers of two whose step stays at or before k
#pragma unroll
            for (u32 step = STEPS; step-- > 0;) {
#pragma unroll
                for (u32 q = 0; q < ATLAS_SPT; ++q) {
                    const u32 k = c0 + threadIdx.x * ATLAS_SPT + q;
                    const u32 probe = found[q] + (1u << step);
                    if (probe < GNB && s.gstart[probe] <= k) found[q] = probe;
                }
            }
#pragma unroll
            for (u32 q = 0; q < ATLAS_SPT; ++q) {
                const u32 k = c0 + threadIdx.x * ATLAS_SPT + q;
                id[q] = 0xFFFFFFFFu;
                gq[q] = 0u;
                if (k < fired_total) {
                    const u32 e = found[q];
                    const u32 g = e / Group::SRC_NB, b = e % Group::SRC_NB, r = k - s.gstart[e];
                    const u32 slot = (u32)((tick - (i64)Group::gval(g)) % Group::SRC_R);
                    id[q] = r < 8 ? small_base[((u64)slot * Group::SRC_NB + b) * 8 + r]
                                  : ids_base[(u64)slot * Group::SRC_N + b * ATLAS_BLOCK + r];
                    gq[q] = g;
                }
            }
            pass(id, gq);
        }
        lds_barrier();
    }
    if constexpr (!Group::COUNT) {
        if (nbuf) flush<Group>(tab, tick, t, blk, nbuf, s, fault);
    }
    if (!hooked) hook();
    lds_barrier();
    if (threadIdx.x < Group::NP && s.delivered[threadIdx.x])
        buf<u64>(tab, Group::DELIVERED)[(u64)Group::path_index(threadIdx.x) * wg_count + wg_index] +=
            s.delivered[threadIdx.x];
    report(tab, Group::FAULT, fault);
    if constexpr (Group::COUNT && APPLY) {
        apply_counts<Group>(tab, tick, t, blk, s);
        lds_barrier();
    }
}

// ---------------------------------------------------------------- persistent tick loop
// One cooperative launch runs `ticks` ticks of a population whose deliveries are one
// counting group of one delay d >= 1 read through complete slot tables (Group), with the
// counted events applied to the updated states in registers (Fused) and the reset fused into
// the update.  The block's states stay in registers for the whole launch.
//
// Tick t is the update (and threshold) U_t, then the deliveries D_t of the spikes of tick
// t - d, applied to the updated states.  U_t needs only the states after tick t - 1, not the
// spikes of t - d, and the slot loads of D_t need only those spikes: so each workgroup first
// waits for the barrier of tick t - d (at which it arrived d ticks earlier), reads the fired
// sources of tick t - d and issues their slot loads, then runs U_t and publishes the spikes of
// tick t while the loads are in flight, and only then counts and applies D_t.  The words of
// each source block are read until they carry the stamp of tick t - d (the barrier says only
// that every block has issued them).  A workgroup that has passed the barrier of tick t - d
// (every block arrived at t - d, so each has read tick t - 2 d, maybe not yet t - 2 d + 1)
// publishes tick t, so the ring holds 2 d + 2 ticks; a wait and the latest arrival span up to
// 2 d barriers, so the barrier counters cycle through 2 d + 2 slots.  Per tick:
//   3. the barrier of tick t - d; the records of tick t - d, one per source block, each read
//      until it carries that tick's stamp; a workgroup scan of their counts; the fired list in
//      LDS (the ids past a record's seventh only marked there);
//   4a. per list entry of the first pass (the marked ones read from the block's id list,
//      likewise stamped) one 32-byte slot load (the source's pathway's), issued back to back
//      by lane pairs, 16 bytes each;
//   1. U_t on the states in registers (Pop::step) with ballots of the fired;
//   2. the fired neurons, ascending, published into the ring (stamped ids; the block's record,
//      its count by thread 0, its first 7 ids by their own work-items) and the recording bitmap;
//      the arrival at the barrier of tick t;
//   4b. integer LDS counts per (pathway, target) from the slots (further passes of a burst
//      loaded and counted the same way);
//   5. each work-item applies its neurons' counts (Fused::apply) in registers and clears them.
// Equal to one launch per tick bit for bit: the same programs in the same order per neuron.
//
// With delay 0 the deliveries of tick t need every block's spikes of tick t, so the tick runs
// U_t, the publication and arrival, then the barrier of tick t, the records, the list, the slot
// loads, the counting and the apply.  A workgroup that has passed the barrier of tick t
// publishes tick t + 1 while the slowest may still read tick t (2 ring slots needed), and it
// can arrive at tick t + 1 before the slowest has seen the barrier of tick t complete, but not
// at tick t + 2 (2 barrier slots).
template <class Pop, class Group, class Fused>
__device__ void persistent_run(const u64* __restrict__ tab, i64 tick0, i64 ticks, u32 blk, u32 nwg,
                               i64 start_tick, double dt_clock, int bar_buf, Lds& s) {
    static_assert(Group::NG == 1 && Group::SLOTS && Group::COUNT, "one delay group through slot tables");
    constexpr u32 HB = Group::HIST_BASE;
    constexpr u32 NP = Group::NP;
    // slot loads per fired source: one when the pathways' source ranges are disjoint (a source is
    // in one pathway at most), else one per pathway
    constexpr u32 ITEMS = Group::DISJOINT ? 1u : NP;
    // fired sources per work-item per pass: 1024 per pass (775 fire per tick in config 3; one
    // slot per work-item of a 1024-wide workgroup measured 0.3 us per tick faster than two)
    constexpr u32 SLOTS_PER = ATLAS_WG >= 1024 ? 1 : 2;
    constexpr u32 LIST = ATLAS_BLOCK;     // fired sources kept in LDS (s.cursor)
    constexpr u32 PERB = (Group::SRC_NB + ATLAS_WG - 1) / ATLAS_WG;   // source blocks per work-item
    constexpr u32 PASS = SLOTS_PER * ATLAS_WG;
    constexpr u32 BAR_SLOTS = 2 * Group::gval_max + 2;   // more than the 2 d barriers a wait and an arrival span
    // delay 0: each tick's deliveries follow its own publication and barrier
    constexpr bool SAME_TICK = Group::gval_max == 0;
    static_assert(Group::SRC_NB <= ATLAS_PASS, "block starts fit s.dense");
    static_assert(Pop::R == Group::SRC_R && Pop::R >= 2 * Group::gval_max + 2 && Pop::R < 4095u &&
                  Pop::R <= ATLAS_RING_PREV, "ring of 2 d + 2 ticks");
    static_assert(Pop::N <= ATLAS_RING_VALUE + 1u, "neuron indices fit a stamped word");
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    const u32 lane = __lane_id();
    const u32 wave = threadIdx.x >> 6;
    const u32 delay = Group::gval(0);
    u32* bar = buf<u32>(tab, bar_buf);
    bool gave_up = false;
    typename Pop::State st[ATLAS_ROUNDS];
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        const u32 j = r * ATLAS_WG + threadIdx.x;
        if (j < n) Pop::load(tab, base + j, st[r]);
    }
    for (u32 j = threadIdx.x; j < NP * ATLAS_BLOCK; j += ATLAS_WG) s.hist[HB + j] = 0;
    // the block's count in each ring slot, as the last publication into it (an earlier launch's,
    // or zero after a reset, which clears the ring) left it
    for (u32 j = threadIdx.x; j < Pop::R; j += ATLAS_WG) s.ring_prev[j] = buf<const u32>(tab, Pop::CNT)[(u64)j * Pop::NB + blk];
    // each work-item's counted events per pathway over the launch, summed over the workgroup once
    // at its end (a per-tick sum measured 0.3 us per tick slower with 4096-neuron blocks)
    u64 lane_delivered[NP];
#pragma unroll
    for (u32 p = 0; p < NP; ++p) lane_delivered[p] = 0;
    // the state loads complete here, before the loop: otherwise the compiler's wait counting
    // assumes they may still be pending on every iteration and waits for every later memory
    // operation before the first use of a state
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    for (i64 k = 0; k < ticks; ++k) {
        const i64 tick = tick0 + k;
        const double t = (double)tick * dt_clock;
        u32 fault = 0;
        const int until_next = Pop::until_next(tab, tick);
        // 3. the fired sources of tick - delay, as every block publishes them
        const i64 emitted = tick - (i64)delay;
        const u32 eslot = (u32)(emitted % Group::SRC_R);
        u32 fired_total = 0;
        auto exchange = [&]() {
        // the exchange (barrier, records, list, slot issue) is the chain every workgroup waits on:
        // its waves take issue priority over another workgroup's update, counting and apply
        __builtin_amdgcn_s_setprio(3);
        if (emitted >= start_tick) {
            // every block has issued its words of tick - delay (those of an earlier launch are
            // ordered by the launch boundary)
            if (emitted >= tick0) grid_wait<BAR_SLOTS>(bar, (u32)(emitted - tick0 + 1), nwg, gave_up, fault);
            const u32 stamp = ring_stamp(emitted);
            uint4 rc[PERB][ATLAS_REC_WORDS / 4];
            u32 local = 0;
#pragma unroll
            for (u32 q = 0; q < PERB; ++q) {
                const u32 b = threadIdx.x * PERB + q;
#pragma unroll
                for (u32 k = 0; k < ATLAS_REC_WORDS / 4; ++k) rc[q][k] = make_uint4(0u, 0u, 0u, 0u);
                if (b < Group::SRC_NB) {
                    ring_wait_record(buf<const u32>(tab, Group::SRC_SMALL) + ((u64)eslot * Group::SRC_NB + b) * ATLAS_REC_WORDS,
                                     stamp, rc[q], gave_up, fault);
                    rc[q][0].x &= ATLAS_RING_VALUE;
                }
                local += rc[q][0].x;
            }
            // exclusive scan of the per-work-item counts: wave scan, wave totals through LDS
            u32 x = local;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const u32 y = __shfl_up(x, off, 64);
                if (lane >= (u32)off) x += y;
            }
            if (lane == 63) s.scan[wave] = x;
            lds_barrier();
            u32 start = x - local;
            for (u32 w = 0; w < ATLAS_WAVES; ++w) {
                const u32 c_ = s.scan[w];
                if (w < wave) start += c_;
                fired_total += c_;
            }
#pragma unroll
            for (u32 q = 0; q < PERB; ++q) {
                const u32 b = threadIdx.x * PERB + q;
                const u32 count = rc[q][0].x;
                if (b < Group::SRC_NB) s.dense[b] = start;   // block starts, for lists that outgrow LDS
                // the ids past the record's are marked and read by the passes below, one per
                // work-item, so a large count costs one round trip instead of one per id
                for (u32 r = 0; r < count; ++r) {
                    const u32 e = start + r;
                    if (e >= LIST) break;   // beyond the LDS list: gathered by the passes below
                    u32 id = ATLAS_LIST_FETCH;
#pragma unroll
                    for (u32 k = 0; k < ATLAS_REC_IDS; ++k)
                        if (r == k) id = record_word(rc[q], k + 1) & ATLAS_RING_VALUE;
                    s.cursor[e] = id;
                }
                start += count;
            }
            lds_barrier();
        }
        };
        // 4a. the first pass's slot loads (one 32-byte load per fired source, or per fired source
        // and pathway where the pathways' source ranges overlap), left in flight under U_t and the
        // publication
        u32 per_path[NP];
#pragma unroll
        for (u32 p = 0; p < NP; ++p) per_path[p] = 0;
        uint4 sa[SLOTS_PER], sb[SLOTS_PER];
        u32 pq[SLOTS_PER];
        auto issue = [&](u32 c0) {
#pragma unroll
            for (u32 q = 0; q < SLOTS_PER; ++q) {
                // item x: fired source e = x / ITEMS, its pathway x % ITEMS when the pathways'
                // source ranges overlap
                const u32 x = c0 + q * ATLAS_WG + threadIdx.x;
                const u32 e = x / ITEMS;
                u32 id = 0xFFFFFFFFu;
                if (e < fired_total) {
                    if (e < LIST) id = s.cursor[e];
                    if (e >= LIST || id == ATLAS_LIST_FETCH) {
                        // an id past a record's seventh, or past the LDS list (a synchronous burst):
                        // the source block is the last whose start is at or before e (binary
                        // search), the id read from its list
                        u32 lo = 0, hi = Group::SRC_NB;
                        while (hi - lo > 1) {
                            const u32 mid = (lo + hi) / 2;
                            if (s.dense[mid] <= e) lo = mid; else hi = mid;
                        }
                        id = ring_wait_u32(buf<const u32>(tab, Group::SRC_IDS) + (u64)eslot * Group::SRC_N +
                                           lo * ATLAS_BLOCK + (e - s.dense[lo]), ring_stamp(emitted), gave_up, fault);
                    }
                }
                // every load issued unconditionally (an entry of no pathway reads the first slot), so
                // they all leave together and nothing waits for one before the next is issued.  The
                // lanes of a pair (2i, 2i + 1) load both their slots, 16 bytes each per slot: one
                // load instruction then touches 32 cache lines instead of 64, which halves the vector
                // cache's tag lookups, the issue rate's limit for these scattered loads
                const uint4* slot = ITEMS == 1 ? Group::source_slot(tab, id, blk, pq[q])
                                               : Group::source_slot_of(tab, id, x % ITEMS, blk, pq[q]);
                const u64 mine = reinterpret_cast<u64>(slot);
                const u64 partner = (u64)lane_swap((u32)mine) | ((u64)lane_swap((u32)(mine >> 32)) << 32);
                const u32 odd = threadIdx.x & 1u;
                // global (not flat) loads: a flat load also counts in the LDS and scalar wait counter,
                // so every later wait for an LDS or scalar value would wait for the slots too
                sa[q] = ((gptr<const uint4>)(odd ? partner : mine))[odd];   // the even lane's slot
                sb[q] = ((gptr<const uint4>)(odd ? mine : partner))[odd];   // the odd lane's slot
            }
        };
        auto count = [&]() {
#pragma unroll
            for (u32 q = 0; q < SLOTS_PER; ++q) {
                // each lane's own slot: the even lane holds its first half and the odd lane's first
                // half, the odd lane both second halves; one swap gives each lane the half it lacks
                const bool odd = threadIdx.x & 1u;
                const uint4 send = odd ? sa[q] : sb[q];
                const uint4 recv = make_uint4(lane_swap(send.x), lane_swap(send.y), lane_swap(send.z),
                                              lane_swap(send.w));
                const uint4 lo = odd ? recv : sa[q], hi = odd ? sb[q] : recv;
                const u32 w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                const bool ok = pq[q] < NP;
                const u32 cnt = ok ? (w[0] & 0xFFFFu) : 0u;
                const u32 inline_cnt = cnt <= 15u ? cnt : 0u;
#pragma unroll
                for (u32 p = 0; p < NP; ++p) per_path[p] += pq[q] == p ? cnt : 0u;
                u32* hist = &s.hist[HB + (ok ? pq[q] : 0u) * ATLAS_BLOCK];
#pragma unroll
                for (u32 r = 0; r < 15; ++r) {
                    if (!__ballot(r < inline_cnt)) break;
                    if (r < inline_cnt) atomicAdd(&hist[(w[(r + 1) / 2] >> (16u * ((r + 1) % 2))) & 0xFFFFu], 1u);
                }
                // a segment longer than the slot's 15 inline targets: read from the row table
                if (__ballot(cnt > 15u) && cnt > 15u) count_long_slot<Group>(tab, pq[q], cnt, w[1], blk, hist);
            }
        };
        if constexpr (!SAME_TICK) {
            exchange();
            issue(0);
            __builtin_amdgcn_s_setprio(0);
        }
        // 1. U_t, under the first pass's slot loads
        u64 masks[ATLAS_ROUNDS];
#pragma unroll
        for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
            const u32 j = r * ATLAS_WG + threadIdx.x;
            bool fired = false;
            if (j < n) fired = Pop::step(tab, base + j, t, tick, st[r], fault, until_next);
            masks[r] = __ballot(fired);
            if (lane == 0) s.round_counts[r * ATLAS_WAVES + wave] = (u32)__popcll(masks[r]);
        }
        lds_barrier();
        // the slot loads are waited for here, before the publication's stores: a store counts in
        // the same counter as a load, so a wait after them would also wait for every store to
        // reach memory
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        // 2. publication of the spikes of tick t, ascending, and the recording bitmap
        {
            const bool recording = Pop::REC >= 0 && tick >= Pop::WIN0;
            const u32 slot = (u32)(tick % Pop::R);
            const u32 stamp = ring_stamp(tick);
            u32* ids = buf<u32>(tab, Pop::IDS) + (u64)slot * Pop::N + base;
            u32* rec = buf<u32>(tab, Pop::SMALL) + ((u64)slot * Pop::NB + blk) * ATLAS_REC_WORDS;
            // each wave's position in the tick's ascending list, per round: the exclusive prefix of
            // the (round, wave) spike counts in round-major order, one count per lane and a wave scan
            // (a loop over the waves' counts per round measured 0.35 us per tick slower with 16 waves)
            static_assert(ATLAS_ROUNDS * ATLAS_WAVES <= 64, "one (round, wave) count per lane");
            const u32 c_ = lane < ATLAS_ROUNDS * ATLAS_WAVES ? s.round_counts[lane] : 0u;
            u32 incl = c_;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const u32 y = __shfl_up(incl, off, 64);
                if (lane >= (u32)off) incl += y;
            }
            const u32 excl = incl - c_;
            const u32 before = __builtin_amdgcn_readlane(incl, 63);
            const u32 wave_u = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
            for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
                const u32 mine = __builtin_amdgcn_readlane(excl, r * ATLAS_WAVES + wave_u);
                if ((masks[r] >> lane) & 1ull) {
                    const u32 kk = mine + (u32)__popcll(masks[r] & ((1ull << lane) - 1ull));
                    const u32 word = ring_word(stamp, base + r * ATLAS_WG + threadIdx.x);
                    ring_store_u32(&ids[kk], word);
                    if (kk < ATLAS_REC_IDS) ring_store_u32(&rec[1 + kk], word);
                }
                if (recording && lane < 2 && r * ATLAS_WG + wave * 64 + lane * 32 < n) {
                    u32* bits = buf<u32>(tab, Pop::REC) + (u64)(tick - Pop::WIN0) * Pop::REC_WORDS;
                    __builtin_nontemporal_store((u32)(masks[r] >> (32 * lane)),
                                                bits + (base + r * ATLAS_WG + wave * 64) / 32 + lane);
                }
            }
            // the words the slot's previous tick wrote past this tick's count (a block that fired
            // fewer neurons now than R ticks ago) are cleared, so that every word of the slot at or
            // past its count is zero and no stale word can carry a later tick's stamp
            const u32 prev = s.ring_prev[slot];
            for (u32 i = before + threadIdx.x; i < prev; i += ATLAS_WG) {
                ring_store_u32(&ids[i], 0u);
                if (i < ATLAS_REC_IDS) ring_store_u32(&rec[1 + i], 0u);
            }
            if (threadIdx.x == 0) {
                ring_store_u32(&rec[0], ring_word(stamp, before));
                buf<u32>(tab, Pop::CNT)[(u64)slot * Pop::NB + blk] = before;   // for the host
            }
            grid_arrive<BAR_SLOTS>(bar, (u32)(k + 1), blk, nwg);
            // every work-item has read the slot's previous count (before grid_arrive's barrier)
            if (threadIdx.x == 0) s.ring_prev[slot] = before;
        }
        if constexpr (SAME_TICK) {
            // delay 0: the tick's own spikes, once every block has published them
            exchange();
            issue(0);
            __builtin_amdgcn_s_setprio(0);
        }
        // 4b. the first pass counted (integer LDS counts per (pathway, target)), then the other
        // passes of a burst loaded and counted
        count();
        for (u32 c0 = PASS; c0 < fired_total * ITEMS; c0 += PASS) {
            issue(c0);
            count();
        }
#pragma unroll
        for (u32 p = 0; p < NP; ++p) lane_delivered[p] += per_path[p];
        lds_barrier();
        // 5. each neuron's counts applied to its updated states, then cleared
#pragma unroll
        for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
            const u32 j = r * ATLAS_WG + threadIdx.x;
            if (j < n) {
                Fused::apply(tab, base + j, j, st[r], s, t, tick, fault);
#pragma unroll
                for (u32 p = 0; p < NP; ++p) s.hist[HB + p * ATLAS_BLOCK + j] = 0;
            }
        }
        report(tab, Pop::FAULT, fault);
    }
    // end of launch: states and delivered counters back to memory
#pragma unroll
    for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {
        const u32 j = r * ATLAS_WG + threadIdx.x;
        if (j < n) Pop::store(tab, base + j, j, st[r], s.post);
    }
    // the launch's delivered events per pathway: wave sums through LDS (the list area is free once
    // the last tick is done), then one work-item per pathway
    static_assert(ATLAS_WAVES * NP * 2 <= ATLAS_PASS, "wave sums fit s.dense");
    lds_barrier();
#pragma unroll
    for (u32 p = 0; p < NP; ++p) {
        u64 v = lane_delivered[p];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) {
            s.dense[2 * (wave * NP + p)] = (u32)v;
            s.dense[2 * (wave * NP + p) + 1] = (u32)(v >> 32);
        }
    }
    lds_barrier();
    u64 delivered = 0;
    if (threadIdx.x < NP)
        for (u32 w = 0; w < ATLAS_WAVES; ++w)
            delivered += (u64)s.dense[2 * (w * NP + threadIdx.x)] | (u64)s.dense[2 * (w * NP + threadIdx.x) + 1] << 32;
    if (threadIdx.x < NP && delivered)
        buf<u64>(tab, Group::DELIVERED)[(u64)Group::path_index(threadIdx.x) * nwg + blk] += delivered;
}

// ---------------------------------------------------------------- split persistent tick loop
// For a delay d >= 1 the counts of tick t need only the spikes of tick t - d, and the update of
// tick t + 1 only the counts of tick t applied.  The split loop runs these two chains side by side
// in one workgroup: its first half of waves (the exchange waves) reads the records of tick t - d
// and counts the events of tick t, while its second half (the update waves, which keep the block's
// states in registers) applies the counts of tick t - 1, runs the update of tick t and publishes
// its spikes.  One workgroup barrier per tick hands the counts over; the LDS counters are
// double-buffered by tick parity.
//
// There is no grid barrier: each exchange wave polls the stamped records of tick t - d of its own
// share of the source blocks until they carry that tick's stamp.  A block publishes tick t only
// after its exchange waves have read every block's records of tick t - 1 - d (their counts come
// before its update), so a block that publishes tick e + R has seen every block publish tick
// e + R - 1 - d, and every block has read tick e before publishing tick e + R - 1 - d when
// R >= 2 d + 2: a ring of 2 d + 2 ticks is never overwritten while read.  Each publication waits
// for the stores of the previous one first (vmcnt(0); they are long complete), so a reader that
// has seen a block's tick e - 1 sees its words of tick e as tick e - R left them or newer: the
// stamp argument of the ring holds as with the barrier.
//
// The first exchange wave only publishes: the update waves leave their fired masks in LDS and
// count themselves in, and that wave writes the block's ascending spike list, record, recording
// bitmap and count as soon as all have arrived.  Every other exchange wave owns up to 64 source
// blocks: one record per lane, a wave scan of the counts, the fired list in the wave's own LDS
// area (no workgroup barrier), then per pass one 32-byte slot load per list entry and lane (two
// passes in flight), counted into the tick's LDS counters with integer atomics.
//
// Measured on config 3 (1M neurons, 245 workgroups of 1024 work-items): 7.8 us per tick for the
// single-chain loop, 6.6 split into halves, 6.0 with the update waves at higher priority and the
// bound checks of full blocks dropped, 5.8 with the masks published by the first exchange wave.
#ifndef ATLAS_XLIST
#define ATLAS_XLIST 512u               // fired sources one exchange wave keeps in LDS per tick
#endif
#ifndef ATLAS_XWAVES
#define ATLAS_XWAVES (ATLAS_WAVES / 2) // exchange waves (the first of the workgroup's waves)
#endif
// Wave priorities of the split loop: the update waves' chain (apply, update) bounds the tick, so
// they issue ahead of the exchange waves, and of two update waves on one SIMD the younger (which
// the hardware would otherwise issue last among equal priorities) goes first.  Measured on config
// 3: 6.6 us per tick with the exchange waves first, 6.0 with the update waves first.
#define ATLAS_XPRIO 0
#define ATLAS_UPRIO_A 1
#define ATLAS_UPRIO_B 2

// Ordered groups (Group::EDGE) replace the counters by the tick's events bucketed by target, in
// ATLAS_SPLIT_HIST words, everything doubled by tick parity: two count arrays of
// ATLAS_EDGE_CNT_WORDS (the exchange waves count a tick's events per target, scan the counts into
// bucket starts and, placing each event, advance them to the bucket ends), then two arrays of
// ATLAS_EDGE_NODES keys and two of as many 8-byte values.
#ifndef ATLAS_SPLIT_HIST
#define ATLAS_SPLIT_HIST (2 * ATLAS_HIST)
#endif
#ifndef ATLAS_EDGE_NODES
#define ATLAS_EDGE_NODES 0u
#endif
#define ATLAS_EDGE_CNT_WORDS (ATLAS_BLOCK + ATLAS_BLOCK / 64u + 4u)
// target j's count word: one pad word per 64, so the scanning wave's lanes (64 consecutive counts
// each) read and write 64 different LDS banks at every step
__device__ __forceinline__ u32 edge_at(u32 j) { return j + (j >> 6); }
#define ATLAS_EDGE_BUCKET_MAX 64u   // events of one target and tick beyond which the tick is replayed

struct LdsSplit {
    u32 ring_prev[ATLAS_RING_PREV];            // the block's count in each ring slot
    u32 pub_done;                              // update waves whose fired masks are in pub_masks
    u32 apply_done;                            // edge buckets: update-wave applications so far
    u32 x_pass;                                // edge buckets: exchange-wave counting passes so far
    u32 x_scan;                                // edge buckets: the last tick (+ 1) whose counts are scanned
    u32 x_bad[2];                              // edge buckets: the tick (by parity) did not fit (replayed)
    u64 pub_masks[64];                         // the tick's fired masks, (round, update wave) order
    u32 wave_sums[2 * ATLAS_WAVES * ATLAS_MAX_NP];
    alignas(16) u32 hist[ATLAS_SPLIT_HIST];    // counters of tick t at (t & 1) * ATLAS_HIST, or edge buckets
    u32 xlist[ATLAS_XWAVES][ATLAS_XLIST];      // each exchange wave's fired list
    u32 xstart[ATLAS_XWAVES][64];              // each exchange wave's block starts in its list
};

// One event of an ordered group in the split loop is keyed pathway << ATLAS_EDGE_BITS | edge id:
// ascending keys are the canonical order of one target's events within a tick (pathways in
// schedule order, then source, then edge).  Its value is the per-edge value its program reads.
#define ATLAS_EDGE_BITS 30u
__device__ __forceinline__ u32* edge_counts(LdsSplit& s, i64 tick) {
    return s.hist + (u32)(tick & 1) * ATLAS_EDGE_CNT_WORDS;
}
__device__ __forceinline__ u32* edge_keys(LdsSplit& s, i64 tick) {
    return s.hist + 2u * ATLAS_EDGE_CNT_WORDS + (u32)(tick & 1) * ATLAS_EDGE_NODES;
}
__device__ __forceinline__ double* edge_values(LdsSplit& s, i64 tick) {
    return reinterpret_cast<double*>(s.hist + 2u * ATLAS_EDGE_CNT_WORDS + 2u * ATLAS_EDGE_NODES) +
           (u32)(tick & 1) * ATLAS_EDGE_NODES;
}

// Waits until an LDS counter of the workgroup reaches `target` (ATLAS_FAULT_STALL after
// ATLAS_SPIN_LIMIT polls, which cannot happen: every wave it counts arrives each tick).
__device__ __forceinline__ void lds_wait_at_least(u32* counter, u32 target, bool& gave_up, u32& fault) {
    u32 spins = 0;
    // a wave that gave up once waits no more, so a stalled launch drains in one spin limit
    while (!gave_up && __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if (++spins >= ATLAS_SPIN_LIMIT) {
            gave_up = true;
            fault |= ATLAS_FAULT_STALL;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One wave turns the block's ATLAS_BLOCK event counts into bucket starts (exclusive scan, in
// place): 64 consecutive counts per lane, then a scan of the lanes' sums.  Returns the total;
// `largest` receives the largest count.
__device__ __forceinline__ u32 edge_scan(u32* cnt, u32& largest) {
    static_assert(ATLAS_BLOCK % 64 == 0, "64 counts per lane");
    constexpr u32 PER = ATLAS_BLOCK / 64;
    const u32 lane = __lane_id();
    u32* mine = cnt + lane * (PER + 1u);
    u32 sum = 0, big = 0;
#pragma unroll 16
    for (u32 i = 0; i < PER; ++i) {
        sum += mine[i];
        big = mine[i] > big ? mine[i] : big;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const u32 y = __shfl_xor(big, off, 64);
        big = y > big ? y : big;
    }
    largest = big;
    u32 x = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const u32 y = __shfl_up(x, off, 64);
        if (lane >= (u32)off) x += y;
    }
    const u32 total = __builtin_amdgcn_readlane(x, 63);
    u32 run = x - sum;
#pragma unroll 16
    for (u32 i = 0; i < PER; ++i) {
        const u32 c = mine[i];
        mine[i] = run;
        run += c;
    }
    return total;
}

// Orders a wave's LDS stores before its lanes' later LDS loads of other lanes' entries.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// The counts of tick `tick` (LDS counters of tick & 1) applied to an update work-item's neurons
// in registers: every count read first, so the LDS reads overlap, then applied and cleared.
template <bool B>
struct BoolTag {
    static constexpr bool value = B;
};

template <class Pop, class Group, class Fused, u32 UR, u32 UL, bool FULL = false>
__device__ __forceinline__ void apply_split(const u64* __restrict__ tab, u32 base, u32 n, u32 ul,
                                            typename Pop::State* st, LdsSplit& s, i64 tick, double dt_clock,
                                            u32& fault) {
    constexpr u32 NP = Group::NP;
    __builtin_assume(ul < UL);
    const u32* h = &s.hist[(u32)(tick & 1) * ATLAS_HIST + Group::HIST_BASE];
    u32 cn[UR][NP];
#pragma unroll
    for (u32 r = 0; r < UR; ++r) {
        const u32 j = r * UL + ul;
#pragma unroll
        for (u32 p = 0; p < NP; ++p) cn[r][p] = (FULL ? j < ATLAS_BLOCK : j < n) ? h[p * ATLAS_BLOCK + j] : 0u;
    }
    const double t = (double)tick * dt_clock;
#pragma unroll
    for (u32 r = 0; r < UR; ++r) {
        const u32 j = r * UL + ul;
        if (FULL ? j < ATLAS_BLOCK : j < n) {
            Fused::apply_n(tab, base + j, st[r], cn[r], t, tick, fault);
#pragma unroll
            for (u32 p = 0; p < NP; ++p) s.hist[(u32)(tick & 1) * ATLAS_HIST + Group::HIST_BASE + p * ATLAS_BLOCK + j] = 0;
        }
    }
}

// One target's bucket [lo, hi) of an edge-keyed tick applied to its states in key order.  Its
// first four entries are sorted by a five-comparator network on (key, position) pairs in
// registers (a bucket of more than four sends every further entry through an insertion that keeps
// the four smallest); they are applied in that order, each value read as it is applied, and a
// bucket of more than four then takes the next smallest key above the last applied, one scan of
// the bucket per event.
template <class Fused, class State>
__device__ __forceinline__ void edge_apply_bucket(const u64* __restrict__ tab, u32 neuron, State& st, const u32* keys,
                                                  const double* vals, u32 lo, u32 hi, double t, i64 tick, u32& fault) {
    const u32 cnt = hi - lo;
    if (!__ballot(cnt != 0u)) return;
    u32 k[4], at[4];
#pragma unroll
    for (u32 i = 0; i < 4; ++i) {
        const bool has = i < cnt;
        at[i] = has ? lo + i : 0u;   // in range either way
        const u32 key = keys[at[i]];
        k[i] = has ? key : ~0u;
    }
    auto cx = [&](u32 a, u32 b) {   // compare-exchange: the smaller key at a
        const bool sw = k[b] < k[a];
        const u32 ka = sw ? k[b] : k[a], kb = sw ? k[a] : k[b];
        const u32 aa = sw ? at[b] : at[a], ab = sw ? at[a] : at[b];
        k[a] = ka;
        k[b] = kb;
        at[a] = aa;
        at[b] = ab;
    };
    cx(0, 1);
    cx(2, 3);
    cx(0, 2);
    cx(1, 3);
    cx(1, 2);
    for (u32 i = 4; __ballot(i < cnt); ++i) {
        if (i < cnt) {
            u32 yk = keys[lo + i], ya = lo + i;
#pragma unroll
            for (u32 m = 0; m < 4; ++m) {
                const bool lt = yk < k[m];
                const u32 tk = lt ? k[m] : yk, ta = lt ? at[m] : ya;
                k[m] = lt ? yk : k[m];
                at[m] = lt ? ya : at[m];
                yk = tk;
                ya = ta;
            }
        }
    }
    u32 last = k[3];
#pragma unroll
    for (u32 i = 0; i < 4; ++i) {
        if (!__ballot(k[i] != ~0u)) break;
        if (k[i] != ~0u) Fused::apply_edge(tab, neuron, st, k[i], vals[at[i]], t, tick, fault);
    }
    u32 left = cnt > 4u ? cnt - 4u : 0u;
    while (__ballot(left != 0u)) {
        u32 best = ~0u, bat = 0u;
        for (u32 i = lo; __ballot(left != 0u && i < hi); ++i) {
            const bool take = left != 0u && i < hi && keys[i] > last && keys[i] < best;
            best = take ? keys[i] : best;
            bat = take ? i : bat;
        }
        if (left) {
            Fused::apply_edge(tab, neuron, st, best, vals[bat], t, tick, fault);
            last = best;
            --left;
        }
    }
}

// The buckets of tick `tick` (counts of tick & 1, advanced to the bucket ends) applied to an
// update work-item's neurons.
template <class Pop, class Fused, u32 UR, u32 UL, bool FULL = false>
__device__ __forceinline__ void apply_split_edges(const u64* __restrict__ tab, u32 base, u32 n, u32 ul,
                                                  typename Pop::State* st, LdsSplit& s, i64 tick, double dt_clock,
                                                  u32& fault) {
    __builtin_assume(ul < UL);
    if (s.x_bad[(u32)(tick & 1)]) return;   // reported; the run is replayed with one launch per tick
    const u32* ends = edge_counts(s, tick);
    const u32* keys = edge_keys(s, tick);
    const double* vals = edge_values(s, tick);
    const double t = (double)tick * dt_clock;
    // the buckets' addresses formed each tick rather than kept live across the tick loop
    u32 ulx = ul;
    asm volatile("" : "+v"(ulx));
#pragma unroll
    for (u32 r = 0; r < UR; ++r) {
        const u32 j = r * UL + ulx;
        const bool in = FULL ? j < ATLAS_BLOCK : j < n;
        u32 hi = in ? ends[edge_at(j)] : 0u;
        u32 lo = (in && j > 0u) ? ends[edge_at(j - 1u)] : 0u;
        hi = hi < ATLAS_EDGE_NODES ? hi : ATLAS_EDGE_NODES;   // a tick past the arrays (reported) applies what fits
        lo = lo < hi ? lo : hi;
        edge_apply_bucket<Fused>(tab, base + j, st[r], keys, vals, lo, hi, t, tick, fault);
    }
}

// The block's spikes of `tick` published by one exchange wave from the update waves' fired masks
// (in LDS once all UW update waves have arrived): lane l holds the mask of round l / UW and update
// wave l % UW, so the exclusive scan of the masks' counts gives ascending list positions; the ids
// and the record's first ids, the recording bitmap, the clearing of the slot's stale words and the
// count word follow.  The stores of the previous publication are waited for first (vmcnt(0)).
template <class Pop, u32 UR, u32 UW, u32 UL>
__device__ __forceinline__ void publish_split(const u64* __restrict__ tab, i64 tick, u32 blk, u32 base, u32 n,
                                              LdsSplit& s, bool& gave_up, u32& fault) {
    static_assert(UR * UW <= 64, "one fired mask per lane");
    const u32 lane = __lane_id();
    u32 spins = 0;
    while (!gave_up && __hip_atomic_load(&s.pub_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < UW) {
        if (++spins >= ATLAS_SPIN_LIMIT) {   // cannot happen: every update wave arrives each tick
            gave_up = true;
            fault |= ATLAS_FAULT_STALL;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the previous publication's stores are complete
    const u32 r = lane / UW, uw = lane % UW;
    const u32 offset = r * UL + uw * 64;   // the mask's first neuron in the block
    u64 m = lane < UR * UW ? s.pub_masks[lane] : 0ull;
    const u32 c = (u32)__popcll(m);
    u32 x = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const u32 y = __shfl_up(x, off, 64);
        if (lane >= (u32)off) x += y;
    }
    const u32 count = __builtin_amdgcn_readlane(x, 63);
    u32 kk = x - c;
    const u32 slot = (u32)(tick % Pop::R);
    const u32 stamp = ring_stamp(tick);
    u32* ids = buf<u32>(tab, Pop::IDS) + (u64)slot * Pop::N + base;
    u32* rec = buf<u32>(tab, Pop::SMALL) + ((u64)slot * Pop::NB + blk) * ATLAS_REC_WORDS;
    while (m) {
        const u32 bit = (u32)__builtin_ctzll(m);
        const u32 word = ring_word(stamp, base + offset + bit);
        ring_store_u32(&ids[kk], word);
        if (kk < ATLAS_REC_IDS) ring_store_u32(&rec[1 + kk], word);
        ++kk;
        m &= m - 1ull;
    }
    if (Pop::REC >= 0 && tick >= Pop::WIN0 && lane < UR * UW && offset < n) {
        const u64 mask = s.pub_masks[lane];
        u32* bits = buf<u32>(tab, Pop::REC) + (u64)(tick - Pop::WIN0) * Pop::REC_WORDS + (base + offset) / 32;
        __builtin_nontemporal_store((u32)mask, bits);
        if (offset + 32 < n) __builtin_nontemporal_store((u32)(mask >> 32), bits + 1);
    }
    // the words the slot's previous tick wrote past this tick's count are cleared, so that every
    // word of the slot at or past its count is zero
    const u32 prev = s.ring_prev[slot];
    for (u32 i = count + lane; i < prev; i += 64) {
        ring_store_u32(&ids[i], 0u);
        if (i < ATLAS_REC_IDS) ring_store_u32(&rec[1 + i], 0u);
    }
    if (lane == 0) {
        ring_store_u32(&rec[0], ring_word(stamp, count));
        buf<u32>(tab, Pop::CNT)[(u64)slot * Pop::NB + blk] = count;   // for the host
        s.ring_prev[slot] = count;
        s.pub_done = 0;
    }
}

template <class Pop, class Group, class Fused>
__device__ __forceinline__ void persistent_run_split(const u64* __restrict__ tab, i64 tick0, i64 ticks, u32 blk, u32 nwg,
                                     i64 start_tick, double dt_clock, LdsSplit& s) {
    static_assert(Group::NG == 1 && (Group::COUNT ? Group::SLOTS : Group::EDGE_SLOTS),
                  "one delay group through slot tables");
    constexpr bool EDGE = !Group::COUNT;             // ordered: edge-keyed buckets instead of counters
    constexpr u32 HB = Group::HIST_BASE;
    constexpr u32 NP = Group::NP;
    constexpr u32 ITEMS = Group::DISJOINT ? 1u : NP;
    constexpr u32 XW = ATLAS_XWAVES;                 // exchange waves
    constexpr u32 UL = ATLAS_WG - 64 * XW;           // update work-items
    constexpr u32 UR = (ATLAS_BLOCK + UL - 1) / UL;  // neurons per update work-item (the last round may be partial)
    constexpr u32 XQ = XW > 1 ? 1u : 0u;             // the first exchange wave only publishes
    constexpr u32 XE = XW - XQ;                      // exchange waves that read records
    constexpr u32 RPW = (Group::SRC_NB + XE - 1) / XE;   // source blocks per exchange wave
    constexpr u32 SP = 2;                            // slot loads in flight per exchange lane
    static_assert(XW >= 1 && XW < ATLAS_WAVES, "exchange and update waves");
    static_assert(RPW <= 64, "one record per exchange lane");
    static_assert(Group::gval_max >= 1, "the counts of a tick need earlier ticks' spikes only");
    static_assert(Pop::R == Group::SRC_R && Pop::R >= 2 * Group::gval_max + 2 && Pop::R < 4095u &&
                  Pop::R <= ATLAS_RING_PREV, "ring of 2 d + 2 ticks");
    static_assert(Pop::N <= ATLAS_RING_VALUE + 1u, "neuron indices fit a stamped word");
    static_assert(EDGE || (HB + NP * ATLAS_BLOCK <= ATLAS_HIST && ATLAS_SPLIT_HIST >= 2 * ATLAS_HIST),
                  "one tick's counters fit a buffer");
    static_assert(!EDGE || (ATLAS_EDGE_NODES > 0 && ATLAS_EDGE_NODES % 2 == 0 &&
                            2 * ATLAS_EDGE_CNT_WORDS + 6 * ATLAS_EDGE_NODES <= ATLAS_SPLIT_HIST && NP <= 4),
                  "edge buckets fit their buffer");
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    const u32 lane = __lane_id();
    const u32 wave = threadIdx.x >> 6;
    const bool xwave = wave < XW;
    const u32 ul = threadIdx.x - 64 * XW;            // update work-item index (update waves)
    const u32 delay = Group::gval(0);
    bool gave_up = false;
    typename Pop::State st[UR];
    if (!xwave) {
#pragma unroll
        for (u32 r = 0; r < UR; ++r) {
            const u32 j = r * UL + ul;
            if (j < n) Pop::load(tab, base + j, st[r]);
        }
    }
    for (u32 j = threadIdx.x; j < ATLAS_SPLIT_HIST; j += ATLAS_WG) s.hist[j] = 0;
    for (u32 j = threadIdx.x; j < Pop::R; j += ATLAS_WG) s.ring_prev[j] = buf<const u32>(tab, Pop::CNT)[(u64)j * Pop::NB + blk];
    if (threadIdx.x == 0) {
        s.pub_done = 0;
        s.apply_done = 0;
        s.x_pass = 0;
        s.x_scan = 0;
        s.x_bad[0] = s.x_bad[1] = 0;
    }
    u64 lane_delivered[NP];
#pragma unroll
    for (u32 p = 0; p < NP; ++p) lane_delivered[p] = 0;
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the state loads, before the loop
    __syncthreads();
    for (i64 k = 0; k < ticks; ++k) {
        const i64 tick = tick0 + k;
        u32 fault = 0;
        if (xwave) {
            // the counts of tick `tick`: the spikes of tick - d, into the counters of tick & 1
            const i64 emitted = tick - (i64)delay;
            const bool active = emitted >= start_tick;
            const u32 xe = wave - XQ;   // this wave's share of the source blocks
            const u32 eslot = active ? (u32)(emitted % Group::SRC_R) : 0u;
            const u32 stamp = ring_stamp(emitted);
            const u32 valid = Group::SRC_NB - xe * RPW < RPW ? Group::SRC_NB - xe * RPW : RPW;
            // the wave's fired list: one record per lane, a wave scan of the counts, the ids in the
            // wave's LDS list (ids past a record's marked, read from the ring below); its length
            auto read_list = [&]() -> u32 {
                const u32 b = xe * RPW + lane;
                const bool mine = lane < RPW && b < Group::SRC_NB;
                uint4 rc[ATLAS_REC_WORDS / 4] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
                if (mine) {
                    ring_wait_record(buf<const u32>(tab, Group::SRC_SMALL) + ((u64)eslot * Group::SRC_NB + b) * ATLAS_REC_WORDS,
                                     stamp, rc, gave_up, fault);
                    rc[0].x &= ATLAS_RING_VALUE;
                }
                const u32 cnt = rc[0].x;
                u32 x = cnt;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const u32 y = __shfl_up(x, off, 64);
                    if (lane >= (u32)off) x += y;
                }
                const u32 total = __builtin_amdgcn_readlane(x, 63);
                const u32 start = x - cnt;
                u32* list = s.xlist[xe];
                if (lane < RPW) s.xstart[xe][lane] = start;
#pragma unroll
                for (u32 r = 0; r < ATLAS_REC_IDS; ++r)
                    if (r < cnt && start + r < ATLAS_XLIST) list[start + r] = record_word(rc, r + 1) & ATLAS_RING_VALUE;
                for (u32 r = ATLAS_REC_IDS; r < cnt && start + r < ATLAS_XLIST; ++r) list[start + r] = ATLAS_LIST_FETCH;
                wave_lds_sync();
                return total;
            };
            // one pass of slot loads: items c0 + q * 64 + lane (q < SP) of the fired list, each
            // lane's slot words handed to handle(pathway, or NP for none, words)
            auto slot_pass = [&](u32 c0, u32 total, auto&& handle) {
                const u32* list = s.xlist[xe];
                uint4 sa[SP], sb[SP];
                u32 pq[SP];
#pragma unroll
                for (u32 q = 0; q < SP; ++q) {
                    const u32 item = c0 + q * 64 + lane;
                    const u32 e = item / ITEMS;
                    u32 id = 0xFFFFFFFFu;
                    if (e < total) {
                        if (e < ATLAS_XLIST) id = list[e];
                        if (e >= ATLAS_XLIST || id == ATLAS_LIST_FETCH) {
                            // the source block is the last of the wave's whose start is at or
                            // before e; the id read from its list
                            u32 lo = 0, hi = valid;
                            while (hi - lo > 1) {
                                const u32 mid = (lo + hi) / 2;
                                if (s.xstart[xe][mid] <= e) lo = mid; else hi = mid;
                            }
                            id = ring_wait_u32(buf<const u32>(tab, Group::SRC_IDS) + (u64)eslot * Group::SRC_N +
                                               (xe * RPW + lo) * ATLAS_BLOCK + (e - s.xstart[xe][lo]), stamp,
                                               gave_up, fault);
                        }
                    }
                    const uint4* slot = ITEMS == 1 ? Group::source_slot(tab, id, blk, pq[q])
                                                   : Group::source_slot_of(tab, id, item % ITEMS, blk, pq[q]);
                    // lane pairs load both their slots, 16 bytes each (every lane active)
                    const u64 mine_ = reinterpret_cast<u64>(slot);
                    const u64 partner = (u64)lane_swap((u32)mine_) | ((u64)lane_swap((u32)(mine_ >> 32)) << 32);
                    const u32 odd = lane & 1u;
                    sa[q] = ((gptr<const uint4>)(odd ? partner : mine_))[odd];
                    sb[q] = ((gptr<const uint4>)(odd ? mine_ : partner))[odd];
                }
#pragma unroll
                for (u32 q = 0; q < SP; ++q) {
                    const bool odd = lane & 1u;
                    const uint4 send = odd ? sa[q] : sb[q];
                    const uint4 recv = make_uint4(lane_swap(send.x), lane_swap(send.y), lane_swap(send.z),
                                                  lane_swap(send.w));
                    const uint4 lo4 = odd ? recv : sa[q], hi4 = odd ? sb[q] : recv;
                    const u32 w[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
                    handle(pq[q], w);
                }
            };
            if constexpr (!EDGE) {
                if (active && wave >= XQ) {
                    __builtin_amdgcn_s_setprio(ATLAS_XPRIO);
                    const u32 total = read_list();
                    u32* hist = &s.hist[(u32)(tick & 1) * ATLAS_HIST + HB];
                    u32 per_path[NP];
#pragma unroll
                    for (u32 p = 0; p < NP; ++p) per_path[p] = 0;
                    for (u32 c0 = 0; c0 < total * ITEMS; c0 += 64 * SP)
                        slot_pass(c0, total, [&](u32 pq, const u32* w) {
                            const bool ok = pq < NP;
                            const u32 c = ok ? (w[0] & 0xFFFFu) : 0u;
#pragma unroll
                            for (u32 p = 0; p < NP; ++p) per_path[p] += pq == p ? c : 0u;
                            const u32 inline_cnt = c <= 15u ? c : 0u;
                            u32* h = &hist[(ok ? pq : 0u) * ATLAS_BLOCK];
#pragma unroll
                            for (u32 r = 0; r < 15; ++r) {
                                if (!__ballot(r < inline_cnt)) break;
                                if (r < inline_cnt) atomicAdd(&h[(w[(r + 1) / 2] >> (16u * ((r + 1) % 2))) & 0xFFFFu], 1u);
                            }
                            if (__ballot(c > 15u) && c > 15u) count_long_slot<Group>(tab, pq, c, w[1], blk, h);
                        });
#pragma unroll
                    for (u32 p = 0; p < NP; ++p) lane_delivered[p] += per_path[p];
                    __builtin_amdgcn_s_setprio(0);
                }
            } else if (wave >= XQ) {
                // edge buckets: the tick's events counted per target, the counts scanned into bucket
                // starts by one wave, then each event placed (key, value) at its bucket's next
                // position.  Row slots: u32 word 1 the segment's first row (= edge id), u16 words
                // 4..15 up to 12 block-local targets (a longer segment's are read from the row table).
                u32* cnt = edge_counts(s, tick);
                __builtin_amdgcn_s_setprio(ATLAS_XPRIO);
                u32 total = 0;
                if (active) {
                    total = read_list();
                    u32 per_path[NP];
#pragma unroll
                    for (u32 p = 0; p < NP; ++p) per_path[p] = 0;
                    for (u32 c0 = 0; c0 < total * ITEMS; c0 += 64 * SP)
                        slot_pass(c0, total, [&](u32 pq, const u32* w) {
                            const bool ok = pq < NP;
                            const u32 c = ok ? (w[0] & 0xFFFFu) : 0u;
#pragma unroll
                            for (u32 p = 0; p < NP; ++p) per_path[p] += pq == p ? c : 0u;
                            const u32 inline_cnt = c <= 12u ? c : 0u;
#pragma unroll
                            for (u32 r = 0; r < 12; ++r) {
                                if (!__ballot(r < inline_cnt)) break;
                                if (r < inline_cnt) atomicAdd(&cnt[edge_at((w[(r + 4) / 2] >> (16u * (r % 2))) & 0xFFFFu)], 1u);
                            }
                            if (__ballot(c > 12u) && c > 12u)
                                for (u32 r = 0; r < c; ++r)
                                    atomicAdd(&cnt[edge_at(Group::row_target(tab, pq, w[1] + r) - blk * ATLAS_BLOCK)], 1u);
                        });
#pragma unroll
                    for (u32 p = 0; p < NP; ++p) lane_delivered[p] += per_path[p];
                }
                // every exchange wave has counted: the first scans
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                if (lane == 0) atomicAdd(&s.x_pass, 1u);
                if (xe == 0) {
                    lds_wait_at_least(&s.x_pass, XE * (u32)(k + 1), gave_up, fault);
                    u32 largest = 0;
                    const u32 events = edge_scan(cnt, largest);
                    // a tick past the arrays, or with a bucket too long to sort in registers, is
                    // reported (the host replays the run with one launch per tick) and not applied
                    const bool bad = events > ATLAS_EDGE_NODES || largest > ATLAS_EDGE_BUCKET_MAX;
                    if (bad) fault |= ATLAS_FAULT_EDGES;
                    if (lane == 0) s.x_bad[(u32)(tick & 1)] = bad ? 1u : 0u;
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                    if (lane == 0) __hip_atomic_store(&s.x_scan, (u32)(k + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
                lds_wait_at_least(&s.x_scan, (u32)(k + 1), gave_up, fault);
                if (active) {
                    u32* keys = edge_keys(s, tick);
                    double* vals = edge_values(s, tick);
                    auto place = [&](u32 target, u32 p, u32 row) {
                        const u32 at = atomicAdd(&cnt[edge_at(target)], 1u);
                        if (at < ATLAS_EDGE_NODES) {
                            keys[at] = p << ATLAS_EDGE_BITS | row;
                            vals[at] = Group::edge_value(tab, p, row);
                        }
                    };
                    for (u32 c0 = 0; c0 < total * ITEMS; c0 += 64 * SP)
                        slot_pass(c0, total, [&](u32 pq, const u32* w) {
                            const bool ok = pq < NP;
                            const u32 c = ok ? (w[0] & 0xFFFFu) : 0u;
                            const u32 pp = ok ? pq : 0u;
                            const u32 inline_cnt = c <= 12u ? c : 0u;
#pragma unroll
                            for (u32 r = 0; r < 12; ++r) {
                                if (!__ballot(r < inline_cnt)) break;
                                if (r < inline_cnt) place((w[(r + 4) / 2] >> (16u * (r % 2))) & 0xFFFFu, pp, w[1] + r);
                            }
                            if (__ballot(c > 12u) && c > 12u)
                                for (u32 r = 0; r < c; ++r)
                                    place(Group::row_target(tab, pp, w[1] + r) - blk * ATLAS_BLOCK, pp, w[1] + r);
                        });
                }
                __builtin_amdgcn_s_setprio(0);
            }
            if (wave == 0) publish_split<Pop, UR, ATLAS_WAVES - XW, UL>(tab, tick, blk, base, n, s, gave_up, fault);
        } else {
          // full blocks (all but possibly the last) bound their neurons by the block size, a
          // constant that removes the checks of every round but a partial last one
          auto utick = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
            __builtin_assume(ul < UL);   // an update work-item (so full rounds need no bound check)
            if (wave - XW < (ATLAS_WAVES - XW) / 2) __builtin_amdgcn_s_setprio(ATLAS_UPRIO_A);
            else __builtin_amdgcn_s_setprio(ATLAS_UPRIO_B);
            const double t = (double)tick * dt_clock;
            const int until_next = Pop::until_next(tab, tick);
            // the counts of tick - 1 (complete since the last barrier) on the states in registers
            if constexpr (EDGE) {
                if (k > 0) apply_split_edges<Pop, Fused, UR, UL, FULL>(tab, base, n, ul, st, s, tick - 1, dt_clock, fault);
                // this wave has read the buckets of tick - 1 (their counts are cleared once all have)
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                if (lane == 0) atomicAdd(&s.apply_done, 1u);
            } else {
                if (k > 0) apply_split<Pop, Group, Fused, UR, UL, FULL>(tab, base, n, ul, st, s, tick - 1, dt_clock, fault);
            }
            // the update of tick
            u64 masks[UR];
#pragma unroll
            for (u32 r = 0; r < UR; ++r) {
                const u32 j = r * UL + ul;
                bool fired = false;
                if (FULL ? j < ATLAS_BLOCK : j < n) fired = Pop::step(tab, base + j, t, tick, st[r], fault, until_next);
                masks[r] = __ballot(fired);
            }
            // the fired masks to LDS, then the arrival the publishing wave waits for
            u32 uw = wave - XW;
            asm volatile("" : "+v"(uw));   // the masks' addresses formed here, not kept live across ticks
#pragma unroll
            for (u32 r = 0; r < UR; ++r)
                if (lane == r) s.pub_masks[r * (ATLAS_WAVES - XW) + uw] = masks[r];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0) atomicAdd(&s.pub_done, 1u);
            if constexpr (EDGE) {
                // once every update wave has read the buckets of tick - 1, their counts are cleared
                // for tick + 1 (the same parity)
                lds_wait_at_least(&s.apply_done, (ATLAS_WAVES - XW) * (u32)(k + 1), gave_up, fault);
                u32* ends = edge_counts(s, tick - 1);
#pragma unroll
                for (u32 r = 0; r < UR; ++r) {
                    const u32 j = r * UL + ul;
                    if (j < ATLAS_BLOCK) ends[edge_at(j)] = 0u;
                }
            }
          };
          // (edge buckets: one instantiation, the bound checks kept, against the code size of two)
          if (!EDGE && n == ATLAS_BLOCK) utick(BoolTag<true>{});
          else utick(BoolTag<false>{});
        }
        report(tab, Pop::FAULT, fault);
        lds_barrier();   // the counts of tick are complete; the publication's LDS words are reset
    }
    // the last tick's counts, then states and delivered counters back to memory
    if (!xwave) {
        u32 fault = 0;
        const i64 last = tick0 + ticks - 1;
        if constexpr (EDGE) {
            if (ticks > 0) apply_split_edges<Pop, Fused, UR, UL>(tab, base, n, ul, st, s, last, dt_clock, fault);
        } else {
            if (ticks > 0) apply_split<Pop, Group, Fused, UR, UL>(tab, base, n, ul, st, s, last, dt_clock, fault);
        }
        report(tab, Pop::FAULT, fault);
#pragma unroll
        for (u32 r = 0; r < UR; ++r) {
            const u32 j = r * UL + ul;
            if (j < n) Pop::store_mem(tab, base + j, st[r]);
        }
    }
#pragma unroll
    for (u32 p = 0; p < NP; ++p) {
        u64 v = lane_delivered[p];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) {
            s.wave_sums[2 * (wave * NP + p)] = (u32)v;
            s.wave_sums[2 * (wave * NP + p) + 1] = (u32)(v >> 32);
        }
    }
    lds_barrier();
    u64 delivered = 0;
    if (threadIdx.x < NP)
        for (u32 w = 0; w < XW; ++w)
            delivered += (u64)s.wave_sums[2 * (w * NP + threadIdx.x)] | (u64)s.wave_sums[2 * (w * NP + threadIdx.x) + 1] << 32;
    if (threadIdx.x < NP && delivered)
        buf<u64>(tab, Group::DELIVERED)[(u64)Group::path_index(threadIdx.x) * nwg + blk] += delivered;
}

// ---------------------------------------------------------------- pushed counts
// Counting groups whose events come with several delays (PUSH groups) are delivered
// by push instead of pull.  In the tick a source fires, its workgroup adds one per
// out-edge to ARR[(tick + delay) % AR][target block][pathway][target] with device-
// scope integer atomics (their order cannot matter), and at the arrival tick each
// target block takes its row of that ring slot into its LDS counters and clears it.
// Pulling would look up the segment of every (fired source, delay group) pair in
// every target block, nearly all of them empty once the delays spread a source's
// edges thin.  The slot written at tick t lies 1..AR-1 ticks ahead, so the row a
// block takes is never written by the same launch.
// Group provides (PUSH groups): AR (largest delay + 1), TB (target blocks), ARR,
// ITEMS (the pathways' delay groups, summed) and push_item(tab, id, i, lo, n, code):
// the rows [lo, lo + n) of the fired source `id`'s i-th (pathway, delay group) and
// code = pathway | delay << 8 (n = 0 when the source is not the pathway's).
template <class Group, class Hook = NoHook>
__device__ void take_counts(const u64* __restrict__ tab, i64 tick, u32 blk, u32 wg_index, u32 wg_count, Lds& s,
                            const Hook& hook = Hook()) {
    constexpr u32 HB = Group::HIST_BASE;
    constexpr u32 ROW = Group::NP * ATLAS_BLOCK;
    constexpr u32 PER = ROW / ATLAS_WG;
    static_assert(ATLAS_BLOCK % ATLAS_WG == 0, "a block is whole rounds of work-items");
    if (threadIdx.x < Group::NP) s.delivered[threadIdx.x] = 0;
    gptr<u32> row = buf<u32>(tab, Group::ARR) + ((u64)(tick % Group::AR) * Group::TB + blk) * ROW;
    u32 c[PER];
#pragma unroll
    for (u32 q = 0; q < PER; ++q) c[q] = row[q * ATLAS_WG + threadIdx.x];
    hook();
    lds_barrier();
    u32 per_path[ATLAS_MAX_NP];
#pragma unroll
    for (u32 p = 0; p < ATLAS_MAX_NP; ++p) per_path[p] = 0;
#pragma unroll
    for (u32 q = 0; q < PER; ++q) {
        const u32 k = q * ATLAS_WG + threadIdx.x;
        s.hist[HB + k] = c[q];
        if (c[q]) row[k] = 0u;
        per_path[q / (ATLAS_BLOCK / ATLAS_WG)] += c[q];
    }
#pragma unroll
    for (u32 p = 0; p < Group::NP; ++p) {
        u32 v = per_path[p];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (__lane_id() == 0 && v) atomicAdd(&s.delivered[p], v);
    }
    if constexpr (Group::PEND_T > 0) {
        lds_barrier();
        count_pending<Group>(tab, tick, blk, s);
    }
    lds_barrier();
    if (threadIdx.x < Group::NP && s.delivered[threadIdx.x])
        buf<u64>(tab, Group::DELIVERED)[(u64)Group::path_index(threadIdx.x) * wg_count + wg_index] +=
            s.delivered[threadIdx.x];
}

// The producer half: called by the workgroup of source block `sblk` once its spikes
// of `tick` are published; edge(code[], row[], valid[]) is called on the out-edges of
// the fired sources, ATLAS_BATCH at a time (code = pathway | delay << 8, valid marks
// the batch's real edges).  The (fired source, pathway, delay group) items are
// spread over the work-items, then their edges: each work-item finds the item of
// its edge by binary search over the items' exclusive starts.
template <class Group, class Edge>
__device__ void push_edges(const u64* __restrict__ tab, i64 tick, u32 sblk, Lds& s, const Edge& edge) {
    static_assert(ATLAS_CAP >= ATLAS_WG && ATLAS_BLOCK >= ATLAS_WG && ATLAS_PASS >= ATLAS_WG,
                  "one LDS entry per work-item");
    static_assert((ATLAS_WG & (ATLAS_WG - 1)) == 0, "power-of-two workgroup");
    const u32 slot = (u32)(tick % Group::SRC_R);
    const u32 fired = buf<const u32>(tab, Group::SRC_CNT)[(u64)slot * Group::SRC_NB + sblk];
    if (fired == 0) return;
    gptr<const u32> ids = buf<const u32>(tab, Group::SRC_IDS) + (u64)slot * Group::SRC_N + sblk * ATLAS_BLOCK;
    const u32 items = fired * Group::ITEMS;
    for (u32 i0 = 0; i0 < items; i0 += ATLAS_WG) {
        const u32 i = i0 + threadIdx.x;
        u32 lo = 0, n = 0, code = 0;
        if (i < items) Group::push_item(tab, ids[i / Group::ITEMS], i % Group::ITEMS, lo, n, code);
        u32 total;
        const u32 first = wg_scan(n, total, s);
        s.dense[threadIdx.x] = first;
        s.ev_row[threadIdx.x] = lo;
        s.cursor[threadIdx.x] = code;
        lds_barrier();
        const u32 last = items - i0 < ATLAS_WG ? items - i0 : ATLAS_WG;
        for (u32 e0 = threadIdx.x; e0 < total; e0 += ATLAS_WG * ATLAS_BATCH) {
            // ATLAS_BATCH edges per work-item at a time, so their memory operations overlap
            u32 code[ATLAS_BATCH], row[ATLAS_BATCH];
            bool valid[ATLAS_BATCH];
#pragma unroll
            for (u32 b = 0; b < ATLAS_BATCH; ++b) {
                const u32 e = e0 + b * ATLAS_WG;
                valid[b] = e < total;
                // the last item starting at or before e (empty items share their start)
                u32 a = 0;
#pragma unroll
                for (u32 step = ATLAS_WG / 2; step > 0; step >>= 1)
                    if (a + step < last && s.dense[a + step] <= e) a += step;
                code[b] = s.cursor[a];
                row[b] = s.ev_row[a] + (e - s.dense[a]);
            }
            edge(code, row, valid);
        }
        lds_barrier();
    }
}

template <class Group>
__device__ void push_counts(const u64* __restrict__ tab, i64 tick, u32 sblk, Lds& s) {
    gptr<u32> arr = buf<u32>(tab, Group::ARR);
    using Batch = u32[ATLAS_BATCH];
    push_edges<Group>(tab, tick, sblk, s, [&](const Batch& code, const Batch& row, const bool (&valid)[ATLAS_BATCH]) {
        u32 tgt[ATLAS_BATCH];
#pragma unroll
        for (u32 b = 0; b < ATLAS_BATCH; ++b)
            if (valid[b]) tgt[b] = Group::row_target(tab, code[b] & 0xFFu, row[b]);
#pragma unroll
        for (u32 b = 0; b < ATLAS_BATCH; ++b) {
            if (!valid[b]) continue;
            const u32 p = code[b] & 0xFFu, d = code[b] >> 8;
            const u64 at = (((u64)((tick + (i64)d) % Group::AR) * Group::TB + tgt[b] / ATLAS_BLOCK) * Group::NP +
                            p) * ATLAS_BLOCK + tgt[b] % ATLAS_BLOCK;
            __hip_atomic_fetch_add(&arr[at], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    });
}

// ---------------------------------------------------------------- queued events
// Ordered groups whose events come with several delays (QUEUE groups) are pushed as
// well: each out-edge of a fired source appends one record to the queue of its
// arrival slot and target block, QBUF[(slot * TB + block) * QCAP + position], with the
// position from a device-scope counter QCNT[slot * TB + block].  A record is the
// event's row (Group::record_row of its out-edge position: rows may be ordered by
// target) and (block-local target | pathway << 12 | delay << 16).  The positions
// follow the atomics' arrival, so the target block restores the canonical order per
// target when it applies them (flush, QUEUE comparator); groups are queued only when
// no target receives more than ATLAS_CAP events per tick, so one target's events
// always share a staging window.  A queue that would pass QCAP sets
// ATLAS_FAULT_QUEUE and drops the record: the host then enlarges the queues and
// runs again.

template <class Group>
__device__ void push_events(const u64* __restrict__ tab, i64 tick, u32 sblk, Lds& s) {
    gptr<u32> qcnt = buf<u32>(tab, Group::QCNT);
    gptr<uint2> queue = buf<uint2>(tab, Group::QBUF);
    u32 fault = 0;
    using Batch = u32[ATLAS_BATCH];
    push_edges<Group>(tab, tick, sblk, s, [&](const Batch& code, const Batch& row, const bool (&valid)[ATLAS_BATCH]) {
        u32 tgt[ATLAS_BATCH], pos[ATLAS_BATCH], rec[ATLAS_BATCH];
        u64 q[ATLAS_BATCH];
#pragma unroll
        for (u32 b = 0; b < ATLAS_BATCH; ++b)
            if (valid[b]) {
                tgt[b] = Group::row_target(tab, code[b] & 0xFFu, row[b]);
                rec[b] = Group::record_row(tab, code[b] & 0xFFu, row[b]);
            }
#pragma unroll
        for (u32 b = 0; b < ATLAS_BATCH; ++b) {
            if (!valid[b]) continue;
            q[b] = (u64)((tick + (i64)(code[b] >> 8)) % Group::AR) * Group::TB + tgt[b] / ATLAS_BLOCK;
            pos[b] = __hip_atomic_fetch_add(&qcnt[q[b]], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (u32 b = 0; b < ATLAS_BATCH; ++b) {
            if (!valid[b]) continue;
            if (pos[b] < Group::QCAP)
                queue[q[b] * Group::QCAP + pos[b]] =
                    make_uint2(rec[b], (tgt[b] % ATLAS_BLOCK) | (code[b] & 0xFu) << 12 | (code[b] >> 8) << 16);
            else
                fault |= ATLAS_FAULT_QUEUE;
        }
    });
    report(tab, Group::FAULT, fault);
}

// Stage one queue record as staging entry e.
__device__ __forceinline__ void stage_record(const uint2 r, u32 e, Lds& s, u32 (&per_path)[ATLAS_MAX_NP]) {
    const u32 p = (r.y >> 12) & 0xFu;
    s.ev_row[e] = r.x;
    s.ev_tgt[e] = (u16)(r.y & 0xFFFu);
    s.ev_key[e] = (u16)((p << ATLAS_CAP_BITS) | e);
    s.ev_d[e] = (u16)(r.y >> 16);
    per_path[p < ATLAS_MAX_NP ? p : 0u] += 1u;
}

// The consumer half: the block's queue of this tick.  Up to ATLAS_CAP records are
// staged as they lie (record k as entry k) and flushed once; the flush restores the
// canonical order per target.  More records are first sorted by target into the
// block's scratch area (QSORT, a counting sort: per-target counts, their scan, a
// scatter), so every window of whole targets holding at most ATLAS_CAP events is a
// contiguous range, staged and flushed in turn.  No target receives more than
// ATLAS_CAP events (host check), so one target's events share a window.  Loads are
// issued ATLAS_CAP / ATLAS_WG at a time per work-item.  The counter is cleared for
// the slot's next use.
template <class Group>
__device__ void take_events(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 wg_index, u32 wg_count,
                            Lds& s) {
    constexpr u32 PERE = ATLAS_CAP / ATLAS_WG;
    constexpr u32 PER = ATLAS_BLOCK / ATLAS_WG;
    u32 fault = 0;
    const u64 q = (u64)(tick % Group::AR) * Group::TB + blk;
    gptr<u32> qcnt = buf<u32>(tab, Group::QCNT);
    gptr<const uint2> queue = buf<const uint2>(tab, Group::QBUF) + q * Group::QCAP;
    if (threadIdx.x < Group::NP) s.delivered[threadIdx.x] = 0;
    for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) s.hist[j] = 0;
    u32 count = qcnt[q];
    if (count > Group::QCAP) count = Group::QCAP;   // overflowed: reported by the producer
    u32 per_path[ATLAS_MAX_NP];
#pragma unroll
    for (u32 p = 0; p < ATLAS_MAX_NP; ++p) per_path[p] = 0;
    if (count <= ATLAS_CAP) {
        uint2 r[PERE];
#pragma unroll
        for (u32 b = 0; b < PERE; ++b) {
            const u32 k = threadIdx.x + b * ATLAS_WG;
            if (k < count) r[b] = queue[k];
        }
#pragma unroll
        for (u32 b = 0; b < PERE; ++b) {
            const u32 k = threadIdx.x + b * ATLAS_WG;
            if (k < count) stage_record(r[b], k, s, per_path);
        }
        lds_barrier();
        if (count) flush<Group>(tab, tick, t, blk, count, s, fault);
    } else if constexpr (ATLAS_TSTART > ATLAS_BLOCK) {
        gptr<uint2> sorted = buf<uint2>(tab, Group::QSORT) + (u64)blk * Group::QCAP;
        for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) s.cursor[j] = 0;
        lds_barrier();
        // events per target
        for (u32 k0 = 0; k0 < count; k0 += ATLAS_CAP) {
            u32 j[PERE];
#pragma unroll
            for (u32 b = 0; b < PERE; ++b) {
                const u32 k = k0 + threadIdx.x + b * ATLAS_WG;
                j[b] = k < count ? queue[k].y & 0xFFFu : ATLAS_BLOCK;
            }
#pragma unroll
            for (u32 b = 0; b < PERE; ++b)
                if (j[b] < ATLAS_BLOCK) atomicAdd(&s.cursor[j[b]], 1u);
        }
        lds_barrier();
        // their exclusive scan: s.tstart[j] = first position of target j, s.tstart[BLOCK] = total
        u32 local = 0;
#pragma unroll
        for (u32 b = 0; b < PER; ++b) local += s.cursor[threadIdx.x * PER + b];
        u32 total;
        u32 at = wg_scan(local, total, s);
#pragma unroll
        for (u32 b = 0; b < PER; ++b) {
            const u32 j = threadIdx.x * PER + b;
            s.tstart[j] = at;
            at += s.cursor[j];
            s.cursor[j] = s.tstart[j];
        }
        if (threadIdx.x == 0) s.tstart[ATLAS_BLOCK] = total;
        lds_barrier();
        // scatter into target order
        for (u32 k0 = 0; k0 < count; k0 += ATLAS_CAP) {
            uint2 r[PERE];
#pragma unroll
            for (u32 b = 0; b < PERE; ++b) {
                const u32 k = k0 + threadIdx.x + b * ATLAS_WG;
                if (k < count) r[b] = queue[k];
            }
#pragma unroll
            for (u32 b = 0; b < PERE; ++b) {
                const u32 k = k0 + threadIdx.x + b * ATLAS_WG;
                const u32 j = r[b].y & 0xFFFu;
                if (k < count && j < ATLAS_BLOCK) sorted[atomicAdd(&s.cursor[j], 1u)] = r[b];
            }
        }
        __syncthreads();   // the scattered records, read by other work-items below
        u32 j0 = 0;
        while (j0 < ATLAS_BLOCK) {
            // the window [j0, j1): the most whole targets from j0 whose events fit
            const u32 base = s.tstart[j0];
            u32 lo = j0 + 1, hi = ATLAS_BLOCK;   // s.tstart[j1] - base <= CAP for j1 in [j0 + 1, lo]
            while (lo < hi) {
                const u32 mid = (lo + hi + 1) >> 1;
                if (s.tstart[mid] - base <= ATLAS_CAP) lo = mid; else hi = mid - 1;
            }
            const u32 j1 = lo;
            u32 n = s.tstart[j1] - base;
            if (n > ATLAS_CAP) {   // one target above the cap: excluded by the host
                n = ATLAS_CAP;
                fault |= ATLAS_FAULT_QUEUE;
            }
            uint2 r[PERE];
#pragma unroll
            for (u32 b = 0; b < PERE; ++b) {
                const u32 e = threadIdx.x + b * ATLAS_WG;
                if (e < n) r[b] = sorted[base + e];
            }
#pragma unroll
            for (u32 b = 0; b < PERE; ++b) {
                const u32 e = threadIdx.x + b * ATLAS_WG;
                if (e < n) stage_record(r[b], e, s, per_path);
            }
            lds_barrier();
            if (n) flush<Group>(tab, tick, t, blk, n, s, fault);
            j0 = j1;
        }
    }
    // every work-item has used the count (barriers since): clear it for the slot's next use
    if (threadIdx.x == 0 && count) qcnt[q] = 0u;
#pragma unroll
    for (u32 p = 0; p < Group::NP; ++p) {
        u32 v = per_path[p];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (__lane_id() == 0 && v) atomicAdd(&s.delivered[p], v);
    }
    lds_barrier();
    if (threadIdx.x < Group::NP && s.delivered[threadIdx.x])
        buf<u64>(tab, Group::DELIVERED)[(u64)Group::path_index(threadIdx.x) * wg_count + wg_index] +=
            s.delivered[threadIdx.x];
    report(tab, Group::FAULT, fault);
}

// ---------------------------------------------------------------- on_post
// PostPath provides: N, NB, R, CNT, IDS (the ring of the synapse's target
// population whose events trigger the pathway: its spikes or a custom event's),
// NG and gval(g) (the delay groups; one for a uniform delay D), TSTART,
// TCOUNT (the synapse's target range), OFF / ROWS (incoming edges of each target
// as row positions, one offsets table per delay group; CONTIGUOUS when these are
// the identity, rows ordered by target), DELIVERED, INDEX (delivered-counter row),
// FAULT and apply(tab, row, t, tick, fault).  An on_post event writes only the
// synapse states of its own edge, so the incoming edges of the block's spiking
// neurons are all independent: they are flattened over the whole workgroup (a
// scan of the spikes' in-degrees gives each spike's first edge, and each
// work-item finds the spike of its edge by binary search), so a spike's ~1000
// edges take a few iterations per work-item instead of one wavefront's dozen.
// The block's targets are this workgroup's, so the tick's on_pre deliveries into
// them (which may write the same edges) are complete once the preceding barrier
// passes; dense / ev_row are free by then.
template <class PostPath>
__device__ void post_events(const u64* __restrict__ tab, i64 tick, double t, const u32* ids, u32 count,
                            u32 wg_index, u32 wg_count, Lds& s, u32 g = 0) {
    const u32* off = buf<const u32>(tab, PostPath::OFF) + (u64)g * (PostPath::TCOUNT + 1);
    const u32* rows = buf<const u32>(tab, PostPath::ROWS);
    u32 fault = 0;
    u64 events = 0;
    for (u32 k0 = 0; k0 < count; k0 += ATLAS_WG) {
        const u32 k = k0 + threadIdx.x;
        u32 lo = 0, degree = 0;
        if (k < count) {
            const u32 j = ids[k] - PostPath::TSTART;   // wraps above TCOUNT when below the range
            if (j < PostPath::TCOUNT) {
                lo = off[j];
                degree = off[j + 1] - lo;
            }
        }
        u32 total;
        const u32 first = wg_scan(degree, total, s);
        s.dense[threadIdx.x] = first;
        s.ev_row[threadIdx.x] = lo;
        lds_barrier();
        const u32 spikes = count - k0 < ATLAS_WG ? count - k0 : ATLAS_WG;
        // ATLAS_BATCH edges per work-item at a time: their row, then their per-edge
        // values, are loaded together before any is applied
        for (u32 e0 = threadIdx.x; e0 < total; e0 += ATLAS_WG * ATLAS_BATCH) {
            u32 row[ATLAS_BATCH];
#pragma unroll
            for (u32 b = 0; b < ATLAS_BATCH; ++b) {
                const u32 e = e0 + b * ATLAS_WG;
                if (e < total) {
                    // the last spike whose first edge is at or before e (spikes without
                    // edges share the next one's start)
                    u32 a = 0, z = spikes;
                    while (z - a > 1) {
                        const u32 mid = (a + z) >> 1;
                        if (s.dense[mid] <= e) a = mid; else z = mid;
                    }
                    const u32 at = s.ev_row[a] + (e - s.dense[a]);
                    row[b] = PostPath::CONTIGUOUS ? at : rows[at];
                }
            }
            typename PostPath::Edge v[ATLAS_BATCH];
#pragma unroll
            for (u32 b = 0; b < ATLAS_BATCH; ++b)
                if (e0 + b * ATLAS_WG < total) PostPath::fetch(tab, row[b], v[b]);
#pragma unroll
            for (u32 b = 0; b < ATLAS_BATCH; ++b)
                if (e0 + b * ATLAS_WG < total) PostPath::apply(tab, row[b], v[b], t, tick, fault);
        }
        events += total;
        lds_barrier();
    }
    if (threadIdx.x == 0 && events)
        atomicAdd(&buf<u64>(tab, PostPath::DELIVERED)[(u64)PostPath::INDEX * wg_count + wg_index], events);
    report(tab, PostPath::FAULT, fault);
}

// The on_post events of the block's neurons whose event came gval(g) ticks ago, for every
// delay group g (one group, D, for a uniform delay): the incoming edges of that group.
template <class PostPath>
__device__ void deliver_post(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 wg_index, u32 wg_count,
                             i64 start_tick, Lds& s) {
    for (u32 g = 0; g < PostPath::NG; ++g) {
        const i64 emitted = tick - (i64)PostPath::gval(g);
        if (emitted < start_tick) continue;
        const u32 slot = (u32)(emitted % PostPath::R);
        const u32 count = buf<const u32>(tab, PostPath::CNT)[(u64)slot * PostPath::NB + blk];
        const u32* ids = buf<const u32>(tab, PostPath::IDS) + (u64)slot * PostPath::N + (u64)blk * ATLAS_BLOCK;
        post_events<PostPath>(tab, tick, t, ids, count, wg_index, wg_count, s, g);
    }
}

// Pending on_post events (a continuation's), before the run's own of the tick: the
// population indices of the block's neurons whose events arrive at this tick (with
// per-edge delays, PEND_EDGES, the rows of the edges whose events arrive), per
// (tick - PEND_START, block) PEND_OFF[k * NB + blk] .. [+ 1] into PEND, in the order given.
template <class PostPath>
__device__ void deliver_post_pending(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 wg_index,
                                     u32 wg_count, Lds& s) {
    const i64 k = tick - PostPath::PEND_START;
    if (k < 0 || k >= (i64)PostPath::PEND_T) return;
    const u32* off = buf<const u32>(tab, PostPath::PEND_OFF) + (u64)k * PostPath::NB + blk;
    if (off[0] == off[1]) return;
    if constexpr (PostPath::PEND_EDGES) {
        // per-edge delays: the listed rows themselves, distinct, so all at once
        const u32* rows = buf<const u32>(tab, PostPath::PEND) + off[0];
        const u32 n = off[1] - off[0];
        u32 fault = 0;
        for (u32 e = threadIdx.x; e < n; e += ATLAS_WG) {
            typename PostPath::Edge v;
            PostPath::fetch(tab, rows[e], v);
            PostPath::apply(tab, rows[e], v, t, tick, fault);
        }
        if (threadIdx.x == 0)
            atomicAdd(&buf<u64>(tab, PostPath::DELIVERED)[(u64)PostPath::INDEX * wg_count + wg_index], (u64)n);
        report(tab, PostPath::FAULT, fault);
        (void)s;
    } else {
        post_events<PostPath>(tab, tick, t, buf<const u32>(tab, PostPath::PEND) + off[0], off[1] - off[0],
                              wg_index, wg_count, s);
    }
    lds_barrier();
}

}  // namespace atlas
