// Procedural projections materialised on the host, as the reference prepares them for its GPU
// engines (brian2_rust/gpu_initialization.py prepare_model, initialisation "rust-host-f64-v0";
// brian2-rust/src/executor.rs:19-188 materialize_projection): the edges of a fixed-in-degree or
// fixed-total rule in the reference's source-major order, and per-edge initializer values with
// the host libm.  The engine then lowers the projection as an explicit topology.  Large
// fixed-in-degree projections without initializers or per-edge delays are built on the device
// instead (atlas_sim_fixed_indegree).
//
// Every loop over edges or targets is split over host threads; each thread's share of the
// counting sort is placed by a prefix over the threads, so the order is the reference's whatever
// the thread count.

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <thread>
#include <vector>

#include "../../include/atlas_sim.h"

namespace {

typedef uint64_t u64;
typedef uint32_t u32;

int prepare_fail(char* err, size_t cap, const char* fmt, ...) {
    if (err && cap) {
        va_list args;
        va_start(args, fmt);
        vsnprintf(err, cap, fmt, args);
        va_end(args);
    }
    return ATLAS_E_HOST;
}

// splitmix64 finaliser with the golden-gamma pre-add (large_topology.rs:54-59)
inline u64 finalise(u64 v) {
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

// draw / bounded / uniform_open / normal of large_topology.rs:60-81
inline u64 edge_draw(u64 seed, u64 stream, u64 edge, u64 attempt) {
    return finalise(seed ^ (stream * 0xd2b74407b1ce6e93ull) ^ (edge * 0x9e3779b97f4a7c15ull) ^
                    (attempt * 0xca5a826395121157ull));
}

inline u64 bounded(u64 seed, u64 stream, u64 edge, u64 upper) {
    return (u64)(((unsigned __int128)edge_draw(seed, stream, edge, 0) * upper) >> 64);
}

inline double uniform_open(u64 seed, u64 stream, u64 edge, u64 attempt) {
    return ((double)(edge_draw(seed, stream, edge, attempt) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

inline double normal(u64 seed, u64 stream, u64 edge, u64 attempt) {
    const double u1 = uniform_open(seed, stream, edge, attempt * 2);
    const double u2 = uniform_open(seed, stream + 1, edge, attempt * 2 + 1);
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

unsigned thread_count(u64 work) {
    unsigned n = std::thread::hardware_concurrency();
    n = std::max(1u, std::min(n, 16u));
    return (unsigned)std::max<u64>(1, std::min<u64>(n, work / 4096 + 1));
}

// Runs body(k, begin, end) over `threads` equal ranges of [0, n).
template <class Body>
void split(u64 n, unsigned threads, Body body) {
    std::vector<std::thread> pool;
    for (unsigned k = 0; k < threads; ++k) {
        const u64 begin = n * k / threads, end = n * (k + 1) / threads;
        pool.emplace_back([=, &body] { body(k, begin, end); });
    }
    for (auto& t : pool) t.join();
}

// The in-degree sources of one target in Floyd's visiting order (large_topology.rs:189-211).
// `marks` is an open-addressing set of at least 2 * indegree slots, cleared on return.
// `used` holds the slots to clear.
template <class Visit>
void floyd_sources(u64 sources, u64 indegree, u64 target, u64 seed, std::vector<u64>& marks, std::vector<u64>& used,
                   Visit visit) {
    const u64 mask = marks.size() - 1;
    used.clear();
    auto contains = [&](u64 v) {
        for (u64 h = (v * 0x9e3779b97f4a7c15ull) >> 20;; ++h) {
            const u64 m = marks[h & mask];
            if (m == 0) return false;
            if (m == v + 1) return true;
        }
    };
    auto insert = [&](u64 v) {
        for (u64 h = (v * 0x9e3779b97f4a7c15ull) >> 20;; ++h) {
            u64& m = marks[h & mask];
            if (m == v + 1) return;
            if (m == 0) {
                m = v + 1;
                used.push_back(h & mask);
                return;
            }
        }
    };
    for (u64 candidate = sources - indegree; candidate < sources; ++candidate) {
        const u64 draw = bounded(seed, 0, target * sources + candidate, candidate + 1);
        const u64 source = contains(draw) ? candidate : draw;
        insert(source);
        visit(source);
    }
    for (u64 slot : used) marks[slot] = 0;
}

// Counting sort of edges by source, stable in generation order: counts[k][s] is thread k's
// number of edges from source s; returns each thread's first position per source.
std::vector<std::vector<u32>> placements(const std::vector<std::vector<u32>>& counts, u64 sources) {
    std::vector<std::vector<u32>> cursor(counts.size(), std::vector<u32>(sources));
    u64 position = 0;
    for (u64 s = 0; s < sources; ++s)
        for (size_t k = 0; k < counts.size(); ++k) {
            cursor[k][s] = (u32)position;
            position += counts[k][s];
        }
    return cursor;
}

}  // namespace

extern "C" int atlas_prepare_fixed_indegree(uint64_t sources, uint64_t targets, uint64_t indegree, uint64_t seed,
                                            uint32_t* source_out, uint32_t* target_out, char* err, size_t cap) {
    // build_fixed_indegree_indices (large_topology.rs:213-261)
    const unsigned __int128 edges = (unsigned __int128)targets * indegree;
    if (sources == 0 || targets == 0 || indegree == 0 || indegree > sources || edges > 0xFFFFFFFFull ||
        (unsigned __int128)targets * sources > (unsigned __int128)UINT64_MAX)
        return prepare_fail(err, cap, "invalid fixed-indegree topology specification");
    if (!source_out || !target_out) return prepare_fail(err, cap, "null output");
    const unsigned threads = thread_count(targets * indegree);
    u64 slots = 2;
    while (slots < 2 * indegree) slots <<= 1;
    std::vector<std::vector<u32>> counts(threads, std::vector<u32>(sources, 0));
    split(targets, threads, [&](unsigned k, u64 begin, u64 end) {
        std::vector<u64> marks(slots, 0), used;
        used.reserve(indegree);
        for (u64 t = begin; t < end; ++t)
            floyd_sources(sources, indegree, t, seed, marks, used, [&](u64 s) { ++counts[k][s]; });
    });
    std::vector<std::vector<u32>> cursor = placements(counts, sources);
    split(targets, threads, [&](unsigned k, u64 begin, u64 end) {
        std::vector<u64> marks(slots, 0), used;
        used.reserve(indegree);
        for (u64 t = begin; t < end; ++t)
            floyd_sources(sources, indegree, t, seed, marks, used, [&](u64 s) {
                const u32 p = cursor[k][s]++;
                source_out[p] = (u32)s;
                target_out[p] = (u32)t;
            });
    });
    return ATLAS_OK;
}

extern "C" int atlas_prepare_fixed_total(uint64_t sources, uint64_t targets, uint64_t edges, uint64_t seed,
                                         uint32_t* source_out, uint32_t* target_out, char* err, size_t cap) {
    // build_fixed_total_indices (large_topology.rs:147-187): with replacement, source-major,
    // each source's edges in generation order
    if (sources == 0 || targets == 0 || edges == 0 || edges > 0xFFFFFFFFull)
        return prepare_fail(err, cap, "invalid fixed-total topology specification");
    if (!source_out || !target_out) return prepare_fail(err, cap, "null output");
    const unsigned threads = thread_count(edges);
    std::vector<std::vector<u32>> counts(threads, std::vector<u32>(sources, 0));
    split(edges, threads, [&](unsigned k, u64 begin, u64 end) {
        for (u64 e = begin; e < end; ++e) ++counts[k][bounded(seed, 0, e, sources)];
    });
    std::vector<std::vector<u32>> cursor = placements(counts, sources);
    split(edges, threads, [&](unsigned k, u64 begin, u64 end) {
        for (u64 e = begin; e < end; ++e) {
            const u64 s = bounded(seed, 0, e, sources);
            const u32 p = cursor[k][s]++;
            source_out[p] = (u32)s;
            target_out[p] = (u32)bounded(seed, 1, e, targets);
        }
    });
    return ATLAS_OK;
}

extern "C" int atlas_prepare_initializer(int kind, uint64_t count, uint64_t seed, uint64_t stream, double minimum,
                                         double maximum, double mean, double std_dev, int has_minimum,
                                         int has_maximum, double* out, char* err, size_t cap) {
    if (!out && count) return prepare_fail(err, cap, "null output");
    if (kind == 0) {
        // materialize_uniform (large_topology.rs:129-142)
        if (!std::isfinite(minimum) || !std::isfinite(maximum) || minimum > maximum)
            return prepare_fail(err, cap, "invalid uniform initializer");
        split(count, thread_count(count), [&](unsigned, u64 begin, u64 end) {
            for (u64 e = begin; e < end; ++e) out[e] = minimum + (maximum - minimum) * uniform_open(seed, stream, e, 0);
        });
        return ATLAS_OK;
    }
    if (kind != 1) return prepare_fail(err, cap, "unknown initializer kind %d", kind);
    // deterministic_clipped_normal (large_topology.rs:87-110)
    if (!std::isfinite(mean) || !std::isfinite(std_dev) || std_dev < 0.0 || (has_minimum && !std::isfinite(minimum)) ||
        (has_maximum && !std::isfinite(maximum)) || (has_minimum && has_maximum && minimum > maximum))
        return prepare_fail(err, cap, "invalid clipped-normal initializer");
    std::vector<unsigned char> exhausted(thread_count(count), 0);
    split(count, (unsigned)exhausted.size(), [&](unsigned k, u64 begin, u64 end) {
        for (u64 e = begin; e < end; ++e) {
            bool found = false;
            for (u64 attempt = 0; attempt < 1000 && !found; ++attempt) {
                const double value = mean + std_dev * normal(seed, stream, e, attempt);
                if ((!has_minimum || value >= minimum) && (!has_maximum || value <= maximum)) {
                    out[e] = value;
                    found = true;
                }
            }
            if (!found) exhausted[k] = 1;
        }
    });
    for (unsigned char x : exhausted)
        if (x) return prepare_fail(err, cap, "clipped-normal rejection limit exceeded");
    return ATLAS_OK;
}
