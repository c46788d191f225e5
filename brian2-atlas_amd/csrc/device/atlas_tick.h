// Hand-written gfx950 building blocks of the Brian2-Atlas tick kernels.
//
// The model-specific parts (state-update / threshold / reset statement bodies and
// the per-event on_pre/on_post programs) are generated from AtlasIR and compiled
// together with this header by hiprtc.  The generated code defines, before this
// header is included:
//   ATLAS_BLOCK   neurons per workgroup block (multiple of ATLAS_WG)
//   ATLAS_CAP     events staged in LDS per delivery flush (<= 65535)
//   ATLAS_MAX_NB  largest source-population block count read by a pathway
//
// Execution model (one workgroup = one block of one population, per tick):
//   phase A  state monitor sample, fused refractory/update/threshold for the
//            block's neurons, ascending spike compaction (wavefront ballot +
//            workgroup scan), publication into the population's spike ring;
//   phase B  delivery of every pathway targeting this population into the
//            block's targets, then the reset of the block's fired neurons.
// Phase B reads spike-ring slots of earlier ticks (delay >= 1) or, for delay-0
// pathways, a slot written by the separate phase-A kernel of the same tick.
//
// Delivery order is the reference order (executor.rs:2292-2382): for each target,
// events apply by emission tick ascending, then source ascending, then edge
// ascending.  Events are gathered into LDS in exactly that order, bucketed by
// target with integer LDS atomics, and each bucket is re-sorted by its canonical
// position before one lane applies it sequentially.  No floating-point atomics.


typedef unsigned int u32;
typedef unsigned long long u64;
typedef long long i64;
typedef unsigned short u16;
typedef unsigned char byte_t;

#define ATLAS_WG 256
#define ATLAS_WAVES (ATLAS_WG / 64)

// Fault bits reported through the fault word (host raises on any set bit).
#define ATLAS_FAULT_NONFINITE 1u
#define ATLAS_FAULT_TIMESTEP 2u
#define ATLAS_FAULT_CAPACITY 4u

namespace atlas {

template <class T>
__device__ __forceinline__ T* buf(const u64* __restrict__ tab, int k) {
    return reinterpret_cast<T*>(tab[k]);
}

struct Lds {
    u32 scan[ATLAS_WAVES + 1];
    u32 misc[4];
    u32 pre[ATLAS_MAX_NB + 1];
    u32 excl[ATLAS_WG];
    u32 lo[ATLAS_WG];
    u32 ev_row[ATLAS_CAP];
    u16 ev_tgt[ATLAS_CAP];
    u16 order[ATLAS_CAP];
    u32 hist[ATLAS_BLOCK];
    u32 cursor[ATLAS_BLOCK];
};

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
    __syncthreads();
    if (threadIdx.x == 0) {
        u32 acc = 0;
        for (int w = 0; w < ATLAS_WAVES; ++w) {
            u32 t = s.scan[w];
            s.scan[w] = acc;
            acc += t;
        }
        s.scan[ATLAS_WAVES] = acc;
    }
    __syncthreads();
    u32 r = s.scan[wave] + x - v;
    total = s.scan[ATLAS_WAVES];
    __syncthreads();
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

__device__ __forceinline__ void finite(double x, u32& fault) {
    if (!__builtin_isfinite(x)) fault |= ATLAS_FAULT_NONFINITE;
}

__device__ __forceinline__ void report(const u64* __restrict__ tab, int fault_buf, u32 fault) {
    if (fault) atomicOr(buf<u32>(tab, fault_buf), fault);
}

// ---------------------------------------------------------------- phase A
// Pop provides: N, NB, R, CNT, IDS, REC (recording bitmap or -1), REC_WORDS,
// WIN0 (first recorded tick), FAULT, record(), update().
template <class Pop>
__device__ void phase_a(const u64* __restrict__ tab, i64 tick, double t, u32 blk, Lds& s) {
    const u32 base = blk * ATLAS_BLOCK;
    const u32 n = (Pop::N - base < ATLAS_BLOCK) ? Pop::N - base : ATLAS_BLOCK;
    Pop::record(tab, tick, base, n);
    __syncthreads();
    const u32 slot = (u32)(tick % Pop::R);
    u32* ids = buf<u32>(tab, Pop::IDS) + (u64)slot * Pop::N + base;
    u32 fault = 0;
    u32 running = 0;
    const u32 lane = __lane_id();
    const u32 wave = threadIdx.x >> 6;
    const bool recording = Pop::REC >= 0 && tick >= Pop::WIN0;
    for (u32 r = 0; r < ATLAS_BLOCK; r += ATLAS_WG) {
        const u32 j = r + threadIdx.x;
        bool fired = false;
        if (j < n) fired = Pop::update(tab, base + j, t, tick, fault);
        const u64 mask = __ballot(fired);
        if (lane == 0) s.scan[wave] = (u32)__popcll(mask);
        if (recording && lane < 2 && r + wave * 64 + lane * 32 < n) {
            u32* rec = buf<u32>(tab, Pop::REC) + (u64)(tick - Pop::WIN0) * Pop::REC_WORDS;
            rec[(base + r + wave * 64) / 32 + lane] = (u32)(mask >> (32 * lane));
        }
        __syncthreads();
        u32 before = running;
        u32 total = running;
        for (u32 w = 0; w < ATLAS_WAVES; ++w) {
            if (w < wave) before += s.scan[w];
            total += s.scan[w];
        }
        if (fired) ids[before + (u32)__popcll(mask & ((1ull << lane) - 1ull))] = base + j;
        running = total;
        __syncthreads();
    }
    if (threadIdx.x == 0) buf<u32>(tab, Pop::CNT)[(u64)slot * Pop::NB + blk] = running;
    report(tab, Pop::FAULT, fault);
}

// ---------------------------------------------------------------- reset
template <class Pop>
__device__ void reset_phase(const u64* __restrict__ tab, i64 tick, double t, u32 blk) {
    const u32 slot = (u32)(tick % Pop::R);
    const u32 count = buf<u32>(tab, Pop::CNT)[(u64)slot * Pop::NB + blk];
    const u32* ids = buf<u32>(tab, Pop::IDS) + (u64)slot * Pop::N + blk * ATLAS_BLOCK;
    u32 fault = 0;
    for (u32 k = threadIdx.x; k < count; k += ATLAS_WG) Pop::reset(tab, ids[k], t, tick, fault);
    report(tab, Pop::FAULT, fault);
}

// ---------------------------------------------------------------- delivery
// Apply the staged events [0, nbuf) to the block's targets in canonical order.
template <class Path>
__device__ void flush(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 nbuf, Lds& s,
                      u32& fault) {
    for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) s.hist[j] = 0;
    __syncthreads();
    for (u32 k = threadIdx.x; k < nbuf; k += ATLAS_WG) atomicAdd(&s.hist[s.ev_tgt[k]], 1u);
    __syncthreads();
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
    __syncthreads();
    for (u32 k = threadIdx.x; k < nbuf; k += ATLAS_WG) {
        u32 pos = atomicAdd(&s.cursor[s.ev_tgt[k]], 1u);
        s.order[pos] = (u16)k;
    }
    __syncthreads();
    for (u32 j = threadIdx.x; j < ATLAS_BLOCK; j += ATLAS_WG) {
        const u32 cnt = s.hist[j];
        if (!cnt) continue;
        u16* ord = &s.order[s.cursor[j] - cnt];
        for (u32 a = 1; a < cnt; ++a) {  // restore canonical order inside the bucket
            u16 key = ord[a];
            u32 b = a;
            while (b > 0 && ord[b - 1] > key) {
                ord[b] = ord[b - 1];
                --b;
            }
            ord[b] = key;
        }
        Path::apply(tab, blk * ATLAS_BLOCK + j, ord, cnt, s.ev_row, t, tick, fault);
    }
    __syncthreads();
}

// Path provides: SRC_N, SRC_NB, SRC_R, SRC_CNT, SRC_IDS, SSTART, SCOUNT, TSTART,
// TCOUNT, D, dval(g), NBT, SEG, ROW_TGT, DELIVERED, PATH_INDEX, FAULT, apply().
template <class Path>
__device__ void deliver(const u64* __restrict__ tab, i64 tick, double t, u32 blk, u32 wg_count,
                        i64 start_tick, Lds& s) {
    const u32 base = blk * ATLAS_BLOCK;
    if (base + ATLAS_BLOCK <= Path::TSTART || base >= Path::TSTART + Path::TCOUNT) return;
    const u32* __restrict__ seg = buf<const u32>(tab, Path::SEG);
    const u32* __restrict__ row_tgt = buf<const u32>(tab, Path::ROW_TGT);
    u32 fault = 0;
    u32 nbuf = 0;
    u64 delivered = 0;
    for (u32 g = 0; g < Path::D; ++g) {
        const i64 emitted = tick - (i64)Path::dval(g);
        if (emitted < start_tick) continue;
        const u32 slot = (u32)(emitted % Path::SRC_R);
        // prefix over the source population's per-block spike counts
        const u32* cnt = buf<const u32>(tab, Path::SRC_CNT) + (u64)slot * Path::SRC_NB;
        constexpr u32 PERB = (Path::SRC_NB + ATLAS_WG - 1) / ATLAS_WG;
        u32 local = 0;
        for (u32 q = 0; q < PERB; ++q) {
            u32 k = threadIdx.x * PERB + q;
            if (k < Path::SRC_NB) local += cnt[k];
        }
        u32 fired_total;
        u32 acc = wg_scan(local, fired_total, s);
        for (u32 q = 0; q < PERB; ++q) {
            u32 k = threadIdx.x * PERB + q;
            if (k < Path::SRC_NB) {
                s.pre[k] = acc;
                acc += cnt[k];
            }
        }
        if (threadIdx.x == 0) s.pre[Path::SRC_NB] = fired_total;
        __syncthreads();
        const u32* ids = buf<const u32>(tab, Path::SRC_IDS) + (u64)slot * Path::SRC_N;
        for (u32 c0 = 0; c0 < fired_total; c0 += ATLAS_WG) {
            const u32 k = c0 + threadIdx.x;
            u32 nev = 0, lo = 0;
            if (k < fired_total) {
                u32 a = 0, b = Path::SRC_NB;  // largest block with pre[block] <= k
                while (b - a > 1) {
                    u32 m = (a + b) >> 1;
                    if (s.pre[m] <= k) a = m; else b = m;
                }
                const u32 src = ids[a * ATLAS_BLOCK + (k - s.pre[a])] - Path::SSTART;
                if (src < Path::SCOUNT) {
                    const u64 at = ((u64)src * Path::D + g) * (Path::NBT + 1) + blk;
                    lo = seg[at];
                    nev = seg[at + 1] - lo;
                }
            }
            u32 chunk_total;
            const u32 ex = wg_scan(nev, chunk_total, s);
            s.excl[threadIdx.x] = ex;
            s.lo[threadIdx.x] = lo;
            __syncthreads();
            for (u32 copied = 0; copied < chunk_total;) {
                const u32 take = (chunk_total - copied < ATLAS_CAP - nbuf) ? chunk_total - copied
                                                                          : ATLAS_CAP - nbuf;
                for (u32 p = threadIdx.x; p < take; p += ATLAS_WG) {
                    const u32 q = copied + p;
                    u32 a = 0, b = ATLAS_WG;  // owner: last thread with excl <= q
                    while (b - a > 1) {
                        u32 m = (a + b) >> 1;
                        if (s.excl[m] <= q) a = m; else b = m;
                    }
                    const u32 row = s.lo[a] + (q - s.excl[a]);
                    s.ev_row[nbuf + p] = row;
                    s.ev_tgt[nbuf + p] = (u16)(row_tgt[row] - base);
                }
                nbuf += take;
                copied += take;
                __syncthreads();
                if (nbuf == ATLAS_CAP) {
                    flush<Path>(tab, tick, t, blk, nbuf, s, fault);
                    delivered += nbuf;
                    nbuf = 0;
                }
            }
        }
    }
    if (nbuf) {
        flush<Path>(tab, tick, t, blk, nbuf, s, fault);
        delivered += nbuf;
    }
    if (threadIdx.x == 0 && delivered)
        buf<u64>(tab, Path::DELIVERED)[(u64)Path::PATH_INDEX * wg_count + blockIdx.x] += delivered;
    report(tab, Path::FAULT, fault);
}

}  // namespace atlas
