/*
 * CPU oracle for the Brian2-Atlas simulation hot path.
 *
 * TEST INFRASTRUCTURE ONLY: this library is the checker for the HIP product
 * path and the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.
 *
 * It restates the execution half of the reference CPU engine `b2-runner`
 * (brian2-rust/src/executor.rs) in plain C; the compile half lives in
 * ir_compile.py.  Every function cites the reference code it follows:
 *
 *   - state arrays, register encoding ........ StateArray executor.rs:338-522
 *   - prepare / run / commit ................. Program executor.rs:5488-5670
 *   - evaluate, casts, integer ops ........... executor.rs:5725-6158
 *   - population update / threshold / reset .. executor.rs:2139-2164, 2949-3006, 4157-4186
 *   - fixed refractory recompute ............. executor.rs:4045-4058, timestep model.rs:981-992
 *   - on_pre / on_post pathway queues ........ run_pathway executor.rs:2292-2382,
 *                                              PathwayQueue executor.rs:6160-6212
 *   - schedule dispatch, clocks .............. Runtime::advance executor.rs:3927-4361
 *   - monitors ............................... executor.rs:3038-3051, 3072-3087
 *   - procedural topology, initializers ...... large_topology.rs:54-261, executor.rs:19-137
 *   - counter RNG ............................ executor.rs:190-323
 *   - result dumps ........................... write_dump executor.rs:3147-3340,
 *                                              write_event_monitor_dump executor.rs:3342-3406
 *
 * Arithmetic is IEEE binary64 with contraction disabled (built with
 * -ffp-contract=off): every expression node is evaluated in an f64 register and
 * rounded to f32 only at storage commits or an explicit f64_to_f32 node, as in
 * the reference.  Transcendentals call the host libm, like Rust's f64 methods.
 *
 * How each part is pinned (tests/test_oracle.py):
 *   - execution semantics, pathway queues and delivery order, fixed refractory,
 *     threshold/reset, spike recording, both dump writers: byte-exact against
 *     the reference-produced dump of tests/fixtures/reference-v1 (155 spikes,
 *     1238 events, per-edge delays 1-4), plus the same-tick three-delay
 *     chronology KAT of test_metal_delays.py:49-93;
 *   - Euler update / delayed delivery / reset order on a recurrent network: an
 *     independent dense f64 evaluation (method of gpu_recurrent.py:54-74) with
 *     exact spikes and the reference's tolerances;
 *   - mix64 (both variants), counter_uniform, uniform_open: the published
 *     splitmix64 output sequences (seeds 0 and 1234567);
 *   - fixed_indegree / fixed_total and the uniform / clipped-normal
 *     initializers: exactly equal to the reference test's own restatement
 *     (draw, uniform, normal, endpoints of test_gpu_initialization.py:29-60,
 *     seed 0x12345678), and the whole model of that test (delay initializers,
 *     floor(delay/dt + 0.5), delivery order) equal to its expected loop; plus
 *     the invariants of large_topology.rs:399-419 and chi-square uniformity;
 *   - counter_normal: the pairing convention of test_gpu_random.py:85-101
 *     (pair = index/2, draws d and d+1, even index takes x1) within that
 *     test's tolerance; counter_binomial (PoissonInput) and counter_poisson:
 *     draw by draw against their mathematical definitions evaluated in
 *     60-digit arithmetic from the counter uniforms (tests/test_oracle_draws.py:
 *     the smallest k with u <= CDF(k) for inversion and its reversed tail, the
 *     restart bound on chosen uniforms, the normal approximation from the
 *     pinned counter_normal, the smallest k whose sum of ln u_i reaches
 *     -lambda, and each PTRS trial's candidate, squeeze and acceptance test with
 *     the exact ln Gamma), equal except at counted ties below the evaluation's
 *     rounding; the reference holds no vectors for these draws;
 *   - transcendental ops (exp, log, ...): the host libm, as Rust's f64 methods
 *     on Linux; the shared atlas_math.h functions are pinned to exactly
 *     rounded decimal values; agreement with another libm is unpinned.
 */
#include <math.h>
#include <stdint.h>
#include "atlas_math.h"  /* the engines' shared exponential (brian2-atlas_amd/csrc/device) */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define LANES 256

/* Exponential functions of vector statements (per neuron, per event): 0 = host
 * libm, as the reference (Rust f64::exp / exp_m1); 1 = the engines' shared
 * correctly rounded implementation (atlas_math.h), which the GPU evaluates
 * bit-identically.  Scalar statements (once per tick) always use the host libm:
 * the HIP engine evaluates them on the host with the same libm. */
static int shared_math = 0;
static int in_vector = 0;
static double math_exp(double x) { return shared_math && in_vector ? atlas_exp(x) : exp(x); }
static double math_expm1(double x) { return shared_math && in_vector ? atlas_expm1(x) : expm1(x); }
static double math_log(double x) { return shared_math && in_vector ? atlas_log(x) : log(x); }

enum dtype { DT_F32, DT_F64, DT_I32, DT_I64, DT_U32, DT_U64, DT_BOOL, DT_INDEX, DT_TICK };
enum input_kind { IN_CONSTANT, IN_TIME, IN_INDEX, IN_STATE, IN_PRE, IN_POST, IN_SYN, IN_PARAM,
                  IN_LASTSPIKE, IN_AVAILABLE, IN_RANDOM, IN_NORMAL };
enum domain { D_NEURON, D_PRE, D_POST, D_EDGE };
enum write_kind { W_NEURON, W_PRE, W_SYN, W_AVAILABLE };
/* Must match OPS in ir_compile.py. */
enum op { OP_NEG, OP_NOT, OP_ABS, OP_ARCCOS, OP_ARCSIN, OP_ARCTAN, OP_CEIL, OP_COS, OP_COSH,
          OP_EXP, OP_EXPM1, OP_EXPREL, OP_FLOOR, OP_TRUNC, OP_ROUND_F32, OP_CAST, OP_INT_UNARY,
          OP_INT_BINARY, OP_TIMESTEP, OP_TICK_OFFSET, OP_LOG, OP_LOG10, OP_LOG1P, OP_SIGN, OP_SIN,
          OP_SINH, OP_SQRT, OP_TAN, OP_TANH, OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_POW, OP_MOD,
          OP_FLOORDIV, OP_EQ, OP_NE, OP_GT, OP_GE, OP_LT, OP_LE, OP_AND, OP_OR, OP_CLIP,
          OP_SELECT, OP_BINOMIAL, OP_POISSON };
enum pop_kind { PK_SUBEXPR, PK_UPDATE, PK_THRESHOLD, PK_REGULAR, PK_RESET, PK_COUNT };

typedef struct {
    uint8_t *results; size_t results_len;
    uint8_t *events; size_t events_len; int has_events;
    uint64_t spike_count, synaptic_events, ticks_run;
    double sim_seconds;
} OracleOutput;

/* ------------------------------------------------------------------ errors */
static char g_err[512];
#define FAIL(...) do { snprintf(g_err, sizeof g_err, __VA_ARGS__); return -1; } while (0)
#define TRY(x) do { if ((x) != 0) return -1; } while (0)

static void *xcalloc(size_t n, size_t size) {
    void *p = calloc(n ? n : 1, size ? size : 1);
    if (!p) { fprintf(stderr, "oracle: out of memory\n"); abort(); }
    return p;
}

/* ------------------------------------------------------------ growable vecs */
typedef struct { size_t *v; size_t n, cap; } VecZ;
static void vz_push(VecZ *a, size_t x) {
    if (a->n == a->cap) { a->cap = a->cap ? a->cap * 2 : 16; a->v = realloc(a->v, a->cap * sizeof *a->v); }
    a->v[a->n++] = x;
}
typedef struct { uint8_t *v; size_t n, cap; } VecB;
static void vb_put(VecB *a, const void *data, size_t bytes) {
    if (a->n + bytes > a->cap) {
        size_t cap = a->cap ? a->cap : 4096;
        while (cap < a->n + bytes) cap *= 2;
        a->v = realloc(a->v, cap); a->cap = cap;
    }
    memcpy(a->v + a->n, data, bytes); a->n += bytes;
}
static void vb_u64(VecB *a, uint64_t x) { vb_put(a, &x, 8); }

/* ------------------------------------------------------------ blob reader */
typedef struct { const uint8_t *p, *end; } Reader;
static uint64_t rd_u(Reader *r) { uint64_t x; memcpy(&x, r->p, 8); r->p += 8; return x; }
static int64_t rd_i(Reader *r) { int64_t x; memcpy(&x, r->p, 8); r->p += 8; return x; }
static double rd_f(Reader *r) { double x; memcpy(&x, r->p, 8); r->p += 8; return x; }
static const uint8_t *rd_raw(Reader *r, size_t *len) {
    *len = (size_t)rd_u(r); const uint8_t *d = r->p; r->p += (*len + 7) / 8 * 8; return d;
}
static double *rd_f64s(Reader *r, size_t *n) {
    size_t len; const uint8_t *d = rd_raw(r, &len); *n = len / 8;
    double *out = xcalloc(*n, 8); memcpy(out, d, len); return out;
}
static uint64_t *rd_u64s(Reader *r, size_t *n) {
    size_t len; const uint8_t *d = rd_raw(r, &len); *n = len / 8;
    uint64_t *out = xcalloc(*n, 8); memcpy(out, d, len); return out;
}

/* ----------------------------------------------------------- state arrays */
/* StateArray (executor.rs:338-522): registers hold f64 values for floats and
 * bools, and the raw two's-complement bits for integers. */
typedef struct { int dtype; size_t len, cap; uint8_t *data; } StateArray;

static size_t dt_size(int dtype) {
    switch (dtype) { case DT_F32: case DT_I32: case DT_U32: return 4; case DT_BOOL: return 1; default: return 8; }
}
static double bits_f64(uint64_t b) { double x; memcpy(&x, &b, 8); return x; }
static uint64_t f64_raw(double x) { uint64_t b; memcpy(&b, &x, 8); return b; }

static double sa_get(const StateArray *a, size_t i) {
    switch (a->dtype) {
    case DT_BOOL: return (double)a->data[i];
    case DT_F32: { float x; memcpy(&x, a->data + 4 * i, 4); return (double)x; }
    case DT_F64: { double x; memcpy(&x, a->data + 8 * i, 8); return x; }
    case DT_I32: case DT_U32: { uint32_t x; memcpy(&x, a->data + 4 * i, 4); return bits_f64((uint64_t)x); }
    default: { uint64_t x; memcpy(&x, a->data + 8 * i, 8); return bits_f64(x); }
    }
}
static void sa_set(StateArray *a, size_t i, double v) {
    switch (a->dtype) {
    case DT_BOOL: a->data[i] = v != 0.0; break;
    case DT_F32: { float x = (float)v; memcpy(a->data + 4 * i, &x, 4); break; }
    case DT_F64: memcpy(a->data + 8 * i, &v, 8); break;
    case DT_I32: case DT_U32: { uint32_t x = (uint32_t)f64_raw(v); memcpy(a->data + 4 * i, &x, 4); break; }
    default: { uint64_t x = f64_raw(v); memcpy(a->data + 8 * i, &x, 8); break; }
    }
}
static void sa_push(StateArray *a, double v) {
    size_t w = dt_size(a->dtype);
    if (a->len == a->cap) { a->cap = a->cap ? a->cap * 2 : 1024; a->data = realloc(a->data, a->cap * w); }
    a->len++; sa_set(a, a->len - 1, v);
}
static void sa_read(Reader *r, StateArray *a) {
    a->dtype = (int)rd_u(r); a->len = (size_t)rd_u(r); a->cap = a->len;
    size_t bytes; const uint8_t *d = rd_raw(r, &bytes);
    a->data = xcalloc(bytes ? bytes : 1, 1); memcpy(a->data, d, bytes);
}

/* ------------------------------------------------------------ counter RNG */
/* executor.rs:190-222: mix64 *without* the golden-gamma pre-add. */
static uint64_t mix64_counter(uint64_t v) {
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
    return v ^ (v >> 31);
}
static double counter_uniform_draw(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index, uint64_t draw) {
    uint64_t c = seed ^ (stream * 0x9e3779b97f4a7c15ULL) ^ (tick * 0xd1b54a32d192ed03ULL)
                 ^ (index * 0x94d049bb133111ebULL) ^ (draw * 0x369dea0f31a53f85ULL);
    return (double)(mix64_counter(c) >> 11) * (1.0 / 9007199254740992.0);
}
static double counter_uniform(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index) {
    return counter_uniform_draw(seed, stream, tick, index, 0);
}
static double counter_normal(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index) {
    uint64_t pair = index / 2, draw = 0;
    for (;;) {
        double x1 = 2.0 * counter_uniform_draw(seed, stream, tick, pair, draw) - 1.0;
        double x2 = 2.0 * counter_uniform_draw(seed, stream, tick, pair, draw + 1) - 1.0;
        double radius = x1 * x1 + x2 * x2;
        if (radius < 1.0 && radius != 0.0) {
            double factor = sqrt(-2.0 * math_log(radius) / radius);
            return factor * ((index & 1) == 0 ? x1 : x2);
        }
        draw += 2;
    }
}
/* One inversion search of counter_binomial (executor.rs:254-266): the x the uniform u selects by
 * sequential search from qn = q^n, or -1 once x passes the restart bound (the caller then draws
 * again).  probability <= 0.5 is the smaller tail, q = 1 - probability. */
static double binomial_search(double u, uint64_t n, double probability, double q, double qn, double bound) {
    uint64_t x = 0; double px = qn;
    for (;;) {
        if (u <= px) return (double)x;
        x += 1;
        if ((double)x > bound) return -1.0;
        u -= px;
        px = ((double)(n - x + 1) * probability * px) / ((double)x * q);
    }
}
/* counter_binomial executor.rs:224-268: the normal approximation when requested and both n p and
 * n (1 - p) exceed 5, else inversion from the smaller tail, restarted with the next draw when the
 * search passes n p + 10 sqrt(n p q + 1) (capped at n). */
static double counter_binomial(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index,
                               uint64_t n, double p, int approximate) {
    if (p <= 0.0) return 0.0;
    if (p >= 1.0) return (double)n;
    double loc = (double)n * p, complement = (double)n * (1.0 - p);
    if (approximate && loc > 5.0 && complement > 5.0)
        return counter_normal(seed, stream, tick, index) * sqrt(loc * (1.0 - p)) + loc;
    int reverse = p > 0.5;
    double probability = reverse ? 1.0 - p : p, q = 1.0 - probability;
    double qn = math_exp((double)n * math_log(q));
    double bound = fmin((double)n, (double)n * probability + 10.0 * sqrt((double)n * probability * q + 1.0));
    for (uint64_t draw = 0;; draw++) {
        double x = binomial_search(counter_uniform_draw(seed, stream, tick, index, draw), n, probability, q, qn, bound);
        if (x >= 0.0) return reverse ? (double)n - x : x;
    }
}
/* log_gamma_positive executor.rs:270-288: Lanczos approximation, g = 7, n = 9. */
static double log_gamma_positive(double value) {
    static const double c[8] = { 676.5203681218851, -1259.1392167224028, 771.3234287776531,
        -176.6150291621406, 12.507343278686905, -0.13857109526572012, 9.984369578019572e-6,
        1.5056327351493116e-7 };
    double z = value - 1.0, x = 0.9999999999998099;
    for (int k = 0; k < 8; k++) x += c[k] / (z + (double)k + 1.0);
    double t = z + 7.5;
    return 0.9189385332046727 + (z + 0.5) * math_log(t) - t + math_log(x);
}
/* One trial of Hoermann's transformed rejection (PTRS, executor.rs:305-322) on the uniforms u (a
 * draw in [0, 1)) and v: the candidate when accepted, else -1. */
static double ptrs_trial(double u, double v, double lambda) {
    double root = sqrt(lambda), b = 0.931 + 2.53 * root, a = -0.059 + 0.02483 * b;
    double inverse_alpha = 1.1239 + 1.1328 / (b - 3.4), squeeze = 0.9277 - 3.6224 / (b - 2.0);
    u -= 0.5;
    double us = 0.5 - fabs(u);
    double candidate = floor((2.0 * a / us + b) * u + lambda + 0.43);
    if (us >= 0.07 && v <= squeeze) return candidate;
    if (candidate < 0.0 || (us < 0.013 && v > us)) return -1.0;
    double left = math_log(v * inverse_alpha / (a / (us * us) + b));
    double right = -lambda + candidate * math_log(lambda) - log_gamma_positive(candidate + 1.0);
    return left <= right ? candidate : -1.0;
}
/* counter_poisson executor.rs:290-323: the product method below 10 (the first sample whose product
 * of draws 0..sample reaches exp(-lambda)), PTRS above on the draw pairs (2 j, 2 j + 1). */
static double counter_poisson(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index, double lambda) {
    if (lambda == 0.0) return 0.0;
    if (!isfinite(lambda) || !(lambda >= 0.0 && lambda <= 1.0e12)) return NAN;
    if (lambda < 10.0) {
        double limit = math_exp(-lambda), product = 1.0; uint64_t sample = 0;
        for (;;) {
            product *= counter_uniform_draw(seed, stream, tick, index, sample);
            if (product <= limit) return (double)sample;
            sample++;
        }
    }
    for (uint64_t draw = 0;; draw += 2) {
        double k = ptrs_trial(counter_uniform_draw(seed, stream, tick, index, draw),
                              counter_uniform_draw(seed, stream, tick, index, draw + 1), lambda);
        if (k >= 0.0) return k;
    }
}

/* ---------------------------------------------- procedural topology RNG */
/* large_topology.rs:54-80: mix64 *with* the golden-gamma pre-add. */
static uint64_t mix64_topology(uint64_t v) {
    v += 0x9e3779b97f4a7c15ULL;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
    return v ^ (v >> 31);
}
static uint64_t topo_draw(uint64_t seed, uint64_t stream, uint64_t edge, uint64_t attempt) {
    return mix64_topology(seed ^ (stream * 0xd2b74407b1ce6e93ULL) ^ (edge * 0x9e3779b97f4a7c15ULL)
                          ^ (attempt * 0xca5a826395121157ULL));
}
static uint64_t topo_bounded(uint64_t seed, uint64_t stream, uint64_t edge, uint64_t upper) {
    return (uint64_t)(((unsigned __int128)topo_draw(seed, stream, edge, 0) * upper) >> 64);
}
static double topo_uniform_open(uint64_t seed, uint64_t stream, uint64_t edge, uint64_t attempt) {
    return ((double)(topo_draw(seed, stream, edge, attempt) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
static double topo_normal(uint64_t seed, uint64_t stream, uint64_t edge, uint64_t attempt) {
    double u1 = topo_uniform_open(seed, stream, edge, attempt * 2);
    double u2 = topo_uniform_open(seed, stream + 1, edge, attempt * 2 + 1);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

typedef struct {
    int kind; uint64_t stream; double minimum, maximum, mean, std; int has_min, has_max;
} Initializer;

static void read_initializer(Reader *r, Initializer *s) {
    s->kind = (int)rd_u(r); s->stream = rd_u(r);
    s->minimum = rd_f(r); s->maximum = rd_f(r); s->mean = rd_f(r); s->std = rd_f(r);
    s->has_min = (int)rd_u(r); s->has_max = (int)rd_u(r);
}
/* materialize_uniform / materialize_clipped_normal (large_topology.rs:95-142). */
static int materialize(const Initializer *s, size_t count, uint64_t seed, double *out) {
    if (s->kind == 0) {
        if (!isfinite(s->minimum) || !isfinite(s->maximum) || s->minimum > s->maximum) FAIL("invalid uniform initializer");
        for (size_t e = 0; e < count; e++)
            out[e] = s->minimum + (s->maximum - s->minimum) * topo_uniform_open(seed, s->stream, e, 0);
        return 0;
    }
    for (size_t e = 0; e < count; e++) {
        int ok = 0;
        for (uint64_t attempt = 0; attempt < 1000; attempt++) {
            double v = s->mean + s->std * topo_normal(seed, s->stream, e, attempt);
            if ((!s->has_min || v >= s->minimum) && (!s->has_max || v <= s->maximum)) { out[e] = v; ok = 1; break; }
        }
        if (!ok) FAIL("clipped-normal rejection limit exceeded");
    }
    return 0;
}

/* build_fixed_indegree_indices (large_topology.rs:189-261): Floyd subset per
 * target, then a source-major counting sort that keeps target order. */
static void floyd_sources(uint64_t n_src, uint64_t indegree, uint64_t target, uint64_t seed,
                          uint8_t *mark, uint64_t *out) {
    for (uint64_t k = 0, candidate = n_src - indegree; candidate < n_src; candidate++, k++) {
        uint64_t logical = target * n_src + candidate;
        uint64_t draw = topo_bounded(seed, 0, logical, candidate + 1);
        uint64_t source = mark[draw] ? candidate : draw;
        mark[source] = 1;
        out[k] = source;
    }
    for (uint64_t k = 0; k < indegree; k++) mark[out[k]] = 0;
}
static int build_fixed_indegree(uint64_t n_src, uint64_t n_tgt, uint64_t indegree, uint64_t seed,
                                size_t **src, size_t **tgt, size_t *edges) {
    uint64_t e = n_tgt * indegree;
    if (!n_src || !n_tgt || !indegree || indegree > n_src || e > 0xFFFFFFFFULL)
        FAIL("invalid fixed-indegree topology specification");
    uint8_t *mark = xcalloc(n_src, 1);
    uint64_t *chosen = xcalloc(indegree, 8);
    size_t *counts = xcalloc(n_src + 1, sizeof(size_t));
    for (uint64_t t = 0; t < n_tgt; t++) {
        floyd_sources(n_src, indegree, t, seed, mark, chosen);
        for (uint64_t k = 0; k < indegree; k++) counts[chosen[k] + 1]++;
    }
    for (uint64_t s = 0; s < n_src; s++) counts[s + 1] += counts[s];
    *src = xcalloc(e, sizeof(size_t)); *tgt = xcalloc(e, sizeof(size_t));
    for (uint64_t t = 0; t < n_tgt; t++) {
        floyd_sources(n_src, indegree, t, seed, mark, chosen);
        for (uint64_t k = 0; k < indegree; k++) {
            size_t pos = counts[chosen[k]]++;
            (*src)[pos] = chosen[k]; (*tgt)[pos] = t;
        }
    }
    *edges = e;
    free(mark); free(chosen); free(counts);
    return 0;
}
/* build_fixed_total_indices (large_topology.rs:148-187): with replacement. */
static int build_fixed_total(uint64_t n_src, uint64_t n_tgt, uint64_t e, uint64_t seed,
                             size_t **src, size_t **tgt, size_t *edges) {
    if (!n_src || !n_tgt || !e || e > 0xFFFFFFFFULL) FAIL("invalid fixed-total topology specification");
    size_t *counts = xcalloc(n_src + 1, sizeof(size_t));
    for (uint64_t k = 0; k < e; k++) counts[topo_bounded(seed, 0, k, n_src) + 1]++;
    for (uint64_t s = 0; s < n_src; s++) counts[s + 1] += counts[s];
    *src = xcalloc(e, sizeof(size_t)); *tgt = xcalloc(e, sizeof(size_t));
    for (uint64_t k = 0; k < e; k++) {
        uint64_t s = topo_bounded(seed, 0, k, n_src);
        size_t pos = counts[s]++;
        (*src)[pos] = s; (*tgt)[pos] = topo_bounded(seed, 1, k, n_tgt);
    }
    *edges = e; free(counts);
    return 0;
}

/* ---------------------------------------------------------------- programs */
typedef struct { uint64_t slot, kind; double cval; uint64_t a, b; const double *param; } Binding;
typedef struct { uint64_t code, left, right; int64_t third, guard; uint64_t output; int64_t p[4]; } Instr;
typedef struct { uint64_t kind, index, reg; } WriteT;

typedef struct {
    size_t nreg; double (*reg)[LANES];
    size_t nb; Binding *b; uint8_t *scalar_random;
    size_t nbroad; uint64_t *broad;
    size_t ns, nv; Instr *scalar, *vector;
    size_t nw; WriteT *w;
    int64_t condition;
    uint64_t tick, seed;
} Program;

typedef struct { double *lastspike; uint8_t *not_refractory; } Refractory;

/* Batch (executor.rs:5674-5704). */
typedef struct { size_t start, len, source, target, source_state, target_state, edge; } Batch;
static Batch batch_neurons(size_t start, size_t len) { Batch b = { start, len, 0, 0, 0, 0, 0 }; return b; }
static size_t batch_index(const Batch *b, int domain, size_t lane) {
    switch (domain) { case D_NEURON: return b->start + lane; case D_PRE: return b->source;
                      case D_POST: return b->target; default: return b->edge; }
}

static void read_program(Reader *r, Program *p, double **tables, uint64_t seed) {
    p->seed = seed;
    p->nreg = (size_t)rd_u(r);
    p->reg = xcalloc(p->nreg, sizeof *p->reg);
    p->nb = (size_t)rd_u(r);
    p->b = xcalloc(p->nb, sizeof *p->b);
    for (size_t k = 0; k < p->nb; k++) {
        Binding *b = &p->b[k];
        b->slot = rd_u(r); b->kind = rd_u(r);
        switch (b->kind) {
        case IN_CONSTANT: b->cval = rd_f(r); b->a = rd_u(r); break;
        case IN_INDEX: case IN_PRE: case IN_POST: case IN_SYN: case IN_AVAILABLE: b->a = rd_u(r); break;
        case IN_STATE: case IN_RANDOM: case IN_NORMAL: b->a = rd_u(r); b->b = rd_u(r); break;
        case IN_PARAM: b->a = rd_u(r); b->b = rd_u(r); b->param = tables[b->a]; break;
        default: break;
        }
    }
    size_t n; uint64_t *sr = rd_u64s(r, &n);
    p->scalar_random = xcalloc(p->nreg, 1);
    for (size_t k = 0; k < n; k++) p->scalar_random[sr[k]] = 1;
    free(sr);
    p->broad = rd_u64s(r, &p->nbroad);
    for (int part = 0; part < 2; part++) {
        size_t count = (size_t)rd_u(r);
        Instr *ins = xcalloc(count, sizeof *ins);
        for (size_t k = 0; k < count; k++) {
            ins[k].code = rd_u(r); ins[k].left = rd_u(r); ins[k].right = rd_u(r);
            ins[k].third = rd_i(r); ins[k].guard = rd_i(r); ins[k].output = rd_u(r);
            for (int q = 0; q < 4; q++) ins[k].p[q] = rd_i(r);
        }
        if (part == 0) { p->ns = count; p->scalar = ins; } else { p->nv = count; p->vector = ins; }
    }
    p->nw = (size_t)rd_u(r);
    p->w = xcalloc(p->nw, sizeof *p->w);
    for (size_t k = 0; k < p->nw; k++) { p->w[k].kind = rd_u(r); p->w[k].index = rd_u(r); p->w[k].reg = rd_u(r); }
    p->condition = rd_i(r);
}

/* timestep (model.rs:981-992): Brian2's truncating tick conversion. */
static int brian_timestep(double time, double dt, uint64_t *out) {
    double steps = (time + 1e-3 * dt) / dt;
    if (!(time >= 0.0 && isfinite(dt) && dt > 0.0 && isfinite(steps) && steps < 9223372036854775808.0))
        FAIL("timestep outside Brian2 int64 range");
    *out = (uint64_t)steps;
    return 0;
}

/* cast_register (executor.rs:5780-5829). */
static int cast_register(double value, int source, int target, double *out) {
    uint64_t raw = f64_raw(value);
    if (target == DT_F64) {
        switch (source) {
        case DT_BOOL: *out = value != 0.0; return 0;
        case DT_F32: case DT_F64: *out = value; return 0;
        case DT_I32: *out = (double)(int32_t)(uint32_t)raw; return 0;
        case DT_I64: *out = (double)(int64_t)raw; return 0;
        case DT_U32: *out = (double)(uint32_t)raw; return 0;
        case DT_U64: *out = (double)raw; return 0;
        default: FAIL("unsupported cast source");
        }
    }
    if (source == DT_I32 || source == DT_I64 || source == DT_U32 || source == DT_U64) {
        __int128 numeric = source == DT_I32 ? (__int128)(int32_t)(uint32_t)raw
                         : source == DT_I64 ? (__int128)(int64_t)raw
                         : source == DT_U32 ? (__int128)(uint32_t)raw : (__int128)raw;
        uint64_t enc;
        switch (target) {
        case DT_I32: enc = (uint32_t)(int32_t)numeric; break;
        case DT_I64: enc = (uint64_t)(int64_t)numeric; break;
        case DT_U32: enc = (uint32_t)numeric; break;
        case DT_U64: enc = (uint64_t)numeric; break;
        default: FAIL("unsupported cast target");
        }
        *out = bits_f64(enc); return 0;
    }
    double numeric;
    if (source == DT_BOOL) numeric = value != 0.0;
    else if (source == DT_F32 || source == DT_F64) numeric = value;
    else FAIL("unsupported cast source");
    /* Rust `as` float->int casts saturate and map NaN to zero. */
    uint64_t enc;
    switch (target) {
    case DT_I32: { int32_t v = isnan(numeric) ? 0 : numeric >= 2147483647.0 ? INT32_MAX
                   : numeric <= -2147483648.0 ? INT32_MIN : (int32_t)numeric; enc = (uint32_t)v; break; }
    case DT_I64: { int64_t v = isnan(numeric) ? 0 : numeric >= 9223372036854775807.0 ? INT64_MAX
                   : numeric <= -9223372036854775808.0 ? INT64_MIN : (int64_t)numeric; enc = (uint64_t)v; break; }
    case DT_U32: { uint32_t v = isnan(numeric) || numeric <= 0.0 ? 0 : numeric >= 4294967295.0 ? UINT32_MAX
                   : (uint32_t)numeric; enc = v; break; }
    case DT_U64: { uint64_t v = isnan(numeric) || numeric <= 0.0 ? 0 : numeric >= 18446744073709551615.0
                   ? UINT64_MAX : (uint64_t)numeric; enc = v; break; }
    default: FAIL("unsupported cast target");
    }
    *out = bits_f64(enc);
    return 0;
}

/* integer_unary_value / integer_binary_value (executor.rs:5831-5930). */
static double int_unary(int dtype, int op, double value) {
    uint64_t raw = f64_raw(value), result;
    if (dtype == DT_I32) {
        uint32_t v = (uint32_t)raw;
        result = op == 0 ? (uint32_t)(0u - v) : (uint32_t)(((int32_t)v < 0) ? 0u - v : v);
    } else {
        result = op == 0 ? (0ULL - raw) : (((int64_t)raw < 0) ? 0ULL - raw : raw);
    }
    return bits_f64(result);
}
static int int_binary(int dtype, int op, double left, double right, double *out) {
    uint64_t la = f64_raw(left), lb = f64_raw(right);
    enum { ADD, SUB, MUL, MOD, FLOORDIV, GT, GE, LT, LE };
    if (dtype == DT_I32 || dtype == DT_I64) {
        int64_t a = dtype == DT_I32 ? (int64_t)(int32_t)(uint32_t)la : (int64_t)la;
        int64_t b = dtype == DT_I32 ? (int64_t)(int32_t)(uint32_t)lb : (int64_t)lb;
        switch (op) {
        case GT: *out = a > b; return 0; case GE: *out = a >= b; return 0;
        case LT: *out = a < b; return 0; case LE: *out = a <= b; return 0;
        default: break;
        }
        int64_t v;
        uint64_t ua = (uint64_t)a, ub = (uint64_t)b;
        if (dtype == DT_I32) {
            int32_t x = (int32_t)a, y = (int32_t)b;
            uint32_t ux = (uint32_t)x, uy = (uint32_t)y;
            switch (op) {
            case ADD: v = (int32_t)(ux + uy); break;
            case SUB: v = (int32_t)(ux - uy); break;
            case MUL: v = (int32_t)(ux * uy); break;
            default: {
                if (y == 0) FAIL(op == MOD ? "integer modulo by zero" : "integer division by zero");
                int32_t q = (x == INT32_MIN && y == -1) ? INT32_MIN : x / y;
                int32_t rem = (x == INT32_MIN && y == -1) ? 0 : x % y;
                int32_t fq = (rem != 0 && ((rem < 0) != (y < 0))) ? (int32_t)((uint32_t)q - 1u) : q;
                v = op == FLOORDIV ? fq : (int32_t)(ux - (uint32_t)fq * uy);
            }
            }
            *out = bits_f64((uint32_t)(int32_t)v);
            return 0;
        }
        switch (op) {
        case ADD: v = (int64_t)(ua + ub); break;
        case SUB: v = (int64_t)(ua - ub); break;
        case MUL: v = (int64_t)(ua * ub); break;
        default: {
            if (b == 0) FAIL(op == MOD ? "integer modulo by zero" : "integer division by zero");
            int64_t q = (a == INT64_MIN && b == -1) ? INT64_MIN : a / b;
            int64_t rem = (a == INT64_MIN && b == -1) ? 0 : a % b;
            int64_t fq = (rem != 0 && ((rem < 0) != (b < 0))) ? (int64_t)((uint64_t)q - 1u) : q;
            v = op == FLOORDIV ? fq : (int64_t)(ua - (uint64_t)fq * ub);
        }
        }
        *out = bits_f64((uint64_t)v);
        return 0;
    }
    uint64_t a = dtype == DT_U32 ? (uint32_t)la : la, b = dtype == DT_U32 ? (uint32_t)lb : lb;
    uint64_t mask = dtype == DT_U32 ? 0xFFFFFFFFULL : ~0ULL, v;
    switch (op) {
    case GT: *out = a > b; return 0; case GE: *out = a >= b; return 0;
    case LT: *out = a < b; return 0; case LE: *out = a <= b; return 0;
    case ADD: v = (a + b) & mask; break;
    case SUB: v = (a - b) & mask; break;
    case MUL: v = (a * b) & mask; break;
    case MOD: if (!b) FAIL("integer modulo by zero"); v = a % b; break;
    default: if (!b) FAIL("integer division by zero"); v = a / b; break;
    }
    *out = bits_f64(v);
    return 0;
}

/* evaluate (executor.rs:5932-6158).  Guarded lanes compute only where the mask
 * is non-zero; every arithmetic result must stay finite. */
static int evaluate(Instr *ins, size_t n, double (*reg)[LANES], size_t len, uint64_t seed, uint64_t tick,
                    const Batch *batch) {
    for (size_t k = 0; k < n; k++) {
        const Instr *in = &ins[k];
        const double *a = reg[in->left], *b = reg[in->right];
        const double *c = in->third >= 0 ? reg[in->third] : NULL;
        const double *g = in->guard >= 0 ? reg[in->guard] : NULL;
        double *o = reg[in->output];
        int valid = 1;
        for (size_t l = 0; l < len; l++) {
            if (in->code == OP_SELECT) { o[l] = g[l] != 0.0 ? a[l] : b[l]; continue; }
            if (g && g[l] == 0.0) continue;
            double x = a[l], y = b[l], r;
            switch (in->code) {
            case OP_NEG: r = -x; break;
            case OP_NOT: r = x == 0.0; break;
            case OP_ABS: r = fabs(x); break;
            case OP_ARCCOS: r = acos(x); break;
            case OP_ARCSIN: r = asin(x); break;
            case OP_ARCTAN: r = atan(x); break;
            case OP_CEIL: r = ceil(x); break;
            case OP_COS: r = cos(x); break;
            case OP_COSH: r = cosh(x); break;
            case OP_EXP: r = math_exp(x); break;
            case OP_EXPM1: r = math_expm1(x); break;
            case OP_EXPREL: r = fabs(x) < 1e-16 ? 1.0 : x > 717.0 ? INFINITY : math_expm1(x) / x; break;
            case OP_FLOOR: r = floor(x); break;
            case OP_TRUNC: r = fabs(x) <= 9007199254740992.0 ? trunc(x) : NAN; break;
            case OP_ROUND_F32: { float f = (float)x; r = isfinite(f) ? (double)f : NAN; break; }
            case OP_CAST: TRY(cast_register(x, (int)(in->p[0] >> 8), (int)(in->p[0] & 0xff), &o[l])); continue;
            case OP_INT_UNARY: o[l] = int_unary((int)(in->p[0] >> 8), (int)(in->p[0] & 0xff), x); continue;
            case OP_INT_BINARY: TRY(int_binary((int)(in->p[0] >> 8), (int)(in->p[0] & 0xff), x, y, &o[l])); continue;
            case OP_TIMESTEP: {
                uint64_t ts; TRY(brian_timestep(x, y, &ts));
                if (ts > 9007199254740992ULL) FAIL("timestep outside exact f64 execution range");
                o[l] = (double)ts; continue;
            }
            case OP_TICK_OFFSET: { r = x + (double)in->p[0]; if (!(fabs(r) <= 9007199254740992.0)) r = NAN; break; }
            case OP_LOG: r = math_log(x); break;
            case OP_LOG10: r = log10(x); break;
            case OP_LOG1P: r = log1p(x); break;
            case OP_SIGN: r = x > 0.0 ? 1.0 : x < 0.0 ? -1.0 : 0.0; break;
            case OP_SIN: r = sin(x); break;
            case OP_SINH: r = sinh(x); break;
            case OP_SQRT: r = sqrt(x); break;
            case OP_TAN: r = tan(x); break;
            case OP_TANH: r = tanh(x); break;
            case OP_ADD: r = x + y; break;
            case OP_SUB: r = x - y; break;
            case OP_MUL: r = x * y; break;
            case OP_DIV: r = x / y; break;
            case OP_POW: r = pow(x, y); break;
            case OP_MOD: r = x - y * floor(x / y); break;
            case OP_FLOORDIV: r = floor(x / y); break;
            case OP_EQ: r = x == y; break;
            case OP_NE: r = x != y; break;
            case OP_GT: r = x > y; break;
            case OP_GE: r = x >= y; break;
            case OP_LT: r = x < y; break;
            case OP_LE: r = x <= y; break;
            case OP_AND: r = x != 0.0 && y != 0.0; break;
            case OP_OR: r = x != 0.0 || y != 0.0; break;
            case OP_CLIP: r = fmin(fmax(x, y), c[l]); break;
            case OP_BINOMIAL: {
                if (!batch) FAIL("binomial in scalar expression");
                if (!(isfinite(x) && x >= 0.0 && x <= 1.0)) FAIL("invalid binomial probability");
                o[l] = counter_binomial(seed, (uint64_t)in->p[0], tick, batch_index(batch, (int)in->p[3], l),
                                        (uint64_t)in->p[1], x, (int)in->p[2]);
                continue;
            }
            case OP_POISSON: {
                if (!batch) FAIL("poisson in scalar expression");
                r = counter_poisson(seed, (uint64_t)in->p[0], tick, batch_index(batch, (int)in->p[1], l), x);
                if (!isfinite(r)) FAIL("invalid poisson lambda");
                break;
            }
            default: FAIL("unknown opcode %llu", (unsigned long long)in->code);
            }
            o[l] = r;
            valid &= isfinite(r) != 0;
        }
        if (!valid) FAIL("non-finite numeric value");
    }
    return 0;
}

/* Program::prepare (executor.rs:5488-5515). */
static int program_prepare(Program *p, double time, uint64_t tick) {
    p->tick = tick;
    for (size_t k = 0; k < p->nb; k++) {
        Binding *b = &p->b[k];
        if (b->kind == IN_CONSTANT) p->reg[b->slot][0] = b->cval;
        else if (b->kind == IN_TIME) p->reg[b->slot][0] = time;
        else if (b->kind == IN_RANDOM && p->scalar_random[b->slot]) p->reg[b->slot][0] = counter_uniform(p->seed, b->a, tick, 0);
        else if (b->kind == IN_NORMAL && p->scalar_random[b->slot]) p->reg[b->slot][0] = counter_normal(p->seed, b->a, tick, 0);
    }
    Batch one = batch_neurons(0, 1);
    TRY(evaluate(p->scalar, p->ns, p->reg, 1, p->seed, p->tick, &one));
    for (size_t k = 0; k < p->nbroad; k++) {
        double v = p->reg[p->broad[k]][0];
        for (size_t l = 0; l < LANES; l++) p->reg[p->broad[k]][l] = v;
    }
    return 0;
}

/* Program::run (executor.rs:5517-5593). */
static int program_run(Program *p, StateArray *states, StateArray *pre, StateArray *post, StateArray *syn,
                       const Refractory *refr, const Batch *batch) {
    size_t len = batch->len;
    for (size_t k = 0; k < p->nb; k++) {
        Binding *b = &p->b[k];
        if (p->scalar_random[b->slot]) continue;
        double *o = p->reg[b->slot];
        switch (b->kind) {
        case IN_STATE:
            if (b->b == D_NEURON) for (size_t l = 0; l < len; l++) o[l] = sa_get(&states[b->a], batch->start + l);
            else { double v = sa_get(&states[b->a], batch_index(batch, (int)b->b, 0)); for (size_t l = 0; l < len; l++) o[l] = v; }
            break;
        case IN_PRE: { double v = sa_get(&pre[b->a], batch->source_state); for (size_t l = 0; l < len; l++) o[l] = v; break; }
        case IN_POST: { double v = sa_get(&post[b->a], batch->target_state); for (size_t l = 0; l < len; l++) o[l] = v; break; }
        case IN_SYN: { double v = sa_get(&syn[b->a], batch->edge); for (size_t l = 0; l < len; l++) o[l] = v; break; }
        case IN_PARAM:
            if (b->b == D_NEURON) memcpy(o, b->param + batch->start, len * sizeof(double));
            else { double v = b->param[batch_index(batch, (int)b->b, 0)]; for (size_t l = 0; l < len; l++) o[l] = v; }
            break;
        case IN_INDEX: for (size_t l = 0; l < len; l++) o[l] = (double)batch_index(batch, (int)b->a, l); break;
        case IN_LASTSPIKE:
            if (!refr) FAIL("missing refractory");
            memcpy(o, refr->lastspike + batch->start, len * sizeof(double));
            break;
        case IN_AVAILABLE:
            if (!refr) FAIL("missing refractory");
            for (size_t l = 0; l < len; l++) {
                size_t idx = b->a == D_POST ? batch->target_state : b->a == D_PRE ? batch->source_state
                           : batch_index(batch, (int)b->a, l);
                o[l] = refr->not_refractory[idx];
            }
            break;
        case IN_RANDOM:
            for (size_t l = 0; l < len; l++) o[l] = counter_uniform(p->seed, b->a, p->tick, batch_index(batch, (int)b->b, l));
            break;
        case IN_NORMAL:
            /* a per-lane draw: the shared-math mode evaluates its log as vector code does */
            in_vector = 1;
            for (size_t l = 0; l < len; l++) o[l] = counter_normal(p->seed, b->a, p->tick, batch_index(batch, (int)b->b, l));
            in_vector = 0;
            break;
        default: break;
        }
    }
    in_vector = 1;
    const int rc = evaluate(p->vector, p->nv, p->reg, len, p->seed, p->tick, batch);
    in_vector = 0;
    return rc;
}

/* commit_neurons / commit_available (executor.rs:5595-5613). */
static void commit_neurons(const Program *p, StateArray *states, size_t start, size_t len) {
    for (size_t k = 0; k < p->nw; k++)
        if (p->w[k].kind == W_NEURON)
            for (size_t l = 0; l < len; l++) sa_set(&states[p->w[k].index], start + l, p->reg[p->w[k].reg][l]);
}
static void commit_available(const Program *p, Refractory *refr, size_t start, size_t len) {
    for (size_t k = 0; k < p->nw; k++)
        if (p->w[k].kind == W_AVAILABLE)
            for (size_t l = 0; l < len; l++) refr->not_refractory[start + l] = p->reg[p->w[k].reg][l] != 0.0;
}
/* commit_event (executor.rs:5625-5672). */
static void commit_event(const Program *p, StateArray *pre, StateArray *post, StateArray *syn,
                         size_t source_neuron, size_t target_neuron, size_t edge) {
    for (size_t k = 0; k < p->nw; k++) {
        double v = p->reg[p->w[k].reg][0];
        switch (p->w[k].kind) {
        case W_NEURON: sa_set(&post[p->w[k].index], target_neuron, v); break;
        case W_PRE: sa_set(&pre[p->w[k].index], source_neuron, v); break;
        case W_SYN: sa_set(&syn[p->w[k].index], edge, v); break;
        default: break;
        }
    }
}

/* --------------------------------------------------------------- runtime */
typedef struct {
    int kind; uint64_t state; double scalar; double *param; int dtype;
} MonitorValue;

/* An EventMonitor (executor.rs:3053-3080): (tick, neuron) of every event and the monitored
 * values of each event's neuron at the monitor's schedule position. */
typedef struct {
    size_t event, n_vars;
    MonitorValue *vals;
    VecZ events;
    StateArray *samples;
} EventMonitor;

typedef struct {
    size_t count, clock, steps, window_steps, n_states, n_events;
    double dt;
    int64_t spike_event;
    StateArray *states;
    int has_refr, fixed_refr; uint64_t period_ticks; Refractory refr;
    size_t n_mon; MonitorValue *mon; StateArray *samples; size_t n_record; uint64_t *record;
    size_t n_tables; double **tables;
    size_t n_prog[PK_COUNT]; Program *prog[PK_COUNT];
    size_t n_code; int64_t (*code)[4];
    size_t tick, end_tick;
    VecZ *fired; VecZ *history; /* history: flattened (tick, neuron) pairs */
    size_t *counts; VecZ last_fired, spikes;
    /* SpikeGeneratorGroup schedule: (tick, neuron) ascending, and its cursor */
    size_t n_gen; uint64_t *gen_ticks, *gen_neurons; size_t gen_cursor;
    size_t n_emon; EventMonitor *emon;
} Population;

typedef struct {
    Program program;
    size_t *offsets, *edges;          /* edge_csr over the endpoint indices */
    VecZ *queue; size_t queue_len;
    int64_t uniform_delay;
    size_t *delay; size_t n_delay;
    uint64_t delivered;
    int is_pre; size_t event_index;
    VecZ active;
} Pathway;

/* A synapse code object: 0 a pathway (its index), 1 the clock-driven state update, 2 a summed
 * variable into state `state` of the source (to_pre) or target population, over the endpoint
 * range [start, start + count), its value the program's register `result`. */
typedef struct {
    uint64_t kind, pathway, to_pre, state, result, start, count;
    Program program;
} SynCode;

typedef struct {
    size_t spop, tpop, sstart, tstart, scount, tcount, n_edges;
    size_t *source, *target;
    size_t n_states; StateArray *states;
    size_t n_tables; double **tables;
    size_t n_path; Pathway *path;
    size_t n_code; SynCode *codes;
} Synapse;

typedef struct { uint64_t op, owner_kind, owner, item, clock; } Node;

typedef struct {
    int lift_budget;
    size_t n_clocks; double *clock_dt; size_t *clock_tick, *clock_end;
    double run_start, run_duration;
    uint64_t seed, neuron_count;
    size_t n_pop; Population *pop;
    size_t n_syn; Synapse *syn;
    size_t n_nodes; Node *nodes;
} Model;

/* edge_csr (executor.rs:6168-6183). */
static void edge_csr(const size_t *indices, size_t n, size_t count, size_t **offsets, size_t **edges) {
    size_t *off = xcalloc(count + 1, sizeof(size_t));
    for (size_t e = 0; e < n; e++) off[indices[e] + 1]++;
    for (size_t k = 0; k < count; k++) off[k + 1] += off[k];
    size_t *next = xcalloc(count + 1, sizeof(size_t));
    memcpy(next, off, count * sizeof(size_t));
    size_t *ed = xcalloc(n, sizeof(size_t));
    for (size_t e = 0; e < n; e++) ed[next[indices[e]]++] = e;
    free(next);
    *offsets = off; *edges = ed;
}

static int load_model(Reader *r, Model *m) {
    m->lift_budget = (int)rd_u(r);
    m->n_clocks = (size_t)rd_u(r);
    m->clock_dt = xcalloc(m->n_clocks, 8); m->clock_tick = xcalloc(m->n_clocks, 8); m->clock_end = xcalloc(m->n_clocks, 8);
    for (size_t c = 0; c < m->n_clocks; c++) {
        m->clock_dt[c] = rd_f(r); m->clock_tick[c] = (size_t)rd_u(r);
        m->clock_end[c] = m->clock_tick[c] + (size_t)rd_u(r);
    }
    m->run_start = rd_f(r); m->run_duration = rd_f(r);
    m->seed = rd_u(r); m->neuron_count = rd_u(r);
    m->n_pop = (size_t)rd_u(r);
    m->pop = xcalloc(m->n_pop, sizeof *m->pop);
    for (size_t pi = 0; pi < m->n_pop; pi++) {
        Population *p = &m->pop[pi];
        p->count = (size_t)rd_u(r); p->clock = (size_t)rd_u(r); p->dt = rd_f(r);
        p->steps = (size_t)rd_u(r); p->window_steps = (size_t)rd_u(r);
        p->n_states = (size_t)rd_u(r);
        p->states = xcalloc(p->n_states, sizeof *p->states);
        for (size_t s = 0; s < p->n_states; s++) sa_read(r, &p->states[s]);
        p->has_refr = (int)rd_u(r);
        if (p->has_refr) {
            p->fixed_refr = (int)rd_u(r); p->period_ticks = rd_u(r);
            size_t n; p->refr.lastspike = rd_f64s(r, &n);
            size_t bytes; const uint8_t *d = rd_raw(r, &bytes);
            p->refr.not_refractory = xcalloc(bytes, 1); memcpy(p->refr.not_refractory, d, bytes);
        }
        p->n_events = (size_t)rd_u(r); p->spike_event = rd_i(r);
        p->gen_ticks = rd_u64s(r, &p->n_gen);
        { size_t n; p->gen_neurons = rd_u64s(r, &n); if (n != p->n_gen) FAIL("generator schedule length mismatch"); }
        p->gen_cursor = 0;
        p->n_mon = (size_t)rd_u(r);
        p->mon = xcalloc(p->n_mon, sizeof *p->mon);
        p->samples = xcalloc(p->n_mon, sizeof *p->samples);
        for (size_t k = 0; k < p->n_mon; k++) {
            MonitorValue *mv = &p->mon[k];
            mv->kind = (int)rd_u(r); mv->dtype = (int)rd_u(r);
            if (mv->kind == 0) mv->state = rd_u(r);
            else if (mv->kind == 1) mv->scalar = rd_f(r);
            else { size_t n; mv->param = rd_f64s(r, &n); }
            p->samples[k].dtype = mv->dtype;
        }
        p->record = rd_u64s(r, &p->n_record);
        (void)rd_u(r); /* has state monitor nodes */
        p->n_emon = (size_t)rd_u(r);
        p->emon = xcalloc(p->n_emon ? p->n_emon : 1, sizeof *p->emon);
        for (size_t k = 0; k < p->n_emon; k++) {
            EventMonitor *em = &p->emon[k];
            em->event = (size_t)rd_u(r); em->n_vars = (size_t)rd_u(r);
            if (em->event >= p->n_events) FAIL("event monitor of an unknown event");
            em->vals = xcalloc(em->n_vars ? em->n_vars : 1, sizeof *em->vals);
            em->samples = xcalloc(em->n_vars ? em->n_vars : 1, sizeof *em->samples);
            for (size_t v = 0; v < em->n_vars; v++) {
                MonitorValue *mv = &em->vals[v];
                mv->kind = (int)rd_u(r); mv->dtype = (int)rd_u(r);
                if (mv->kind == 0) mv->state = rd_u(r);
                else if (mv->kind == 1) mv->scalar = rd_f(r);
                else { size_t n; mv->param = rd_f64s(r, &n); }
                em->samples[v].dtype = mv->dtype;
            }
        }
        p->n_tables = (size_t)rd_u(r);
        p->tables = xcalloc(p->n_tables, sizeof *p->tables);
        for (size_t k = 0; k < p->n_tables; k++) { size_t n; p->tables[k] = rd_f64s(r, &n); }
        for (int kind = 0; kind < PK_COUNT; kind++) {
            p->n_prog[kind] = (size_t)rd_u(r);
            p->prog[kind] = xcalloc(p->n_prog[kind], sizeof(Program));
            for (size_t k = 0; k < p->n_prog[kind]; k++) read_program(r, &p->prog[kind][k], p->tables, m->seed);
        }
        p->n_code = (size_t)rd_u(r);
        p->code = xcalloc(p->n_code, sizeof *p->code);
        for (size_t k = 0; k < p->n_code; k++) for (int q = 0; q < 4; q++) p->code[k][q] = rd_i(r);
        p->tick = m->clock_tick[p->clock];
        p->end_tick = p->tick + p->steps;
        p->fired = xcalloc(p->n_events ? p->n_events : 1, sizeof(VecZ));
        p->history = xcalloc(p->n_events ? p->n_events : 1, sizeof(VecZ));
        p->counts = xcalloc(p->count, sizeof(size_t));
    }
    m->n_syn = (size_t)rd_u(r);
    m->syn = xcalloc(m->n_syn, sizeof *m->syn);
    for (size_t si = 0; si < m->n_syn; si++) {
        Synapse *s = &m->syn[si];
        s->spop = (size_t)rd_u(r); s->tpop = (size_t)rd_u(r);
        s->sstart = (size_t)rd_u(r); s->tstart = (size_t)rd_u(r);
        s->scount = (size_t)rd_u(r); s->tcount = (size_t)rd_u(r);
        uint64_t topo = rd_u(r);
        size_t n_init = 0; Initializer *inits = NULL; uint64_t tseed = 0;
        if (topo == 0) {
            size_t n1, n2; uint64_t *src = rd_u64s(r, &n1), *tgt = rd_u64s(r, &n2);
            s->n_edges = n1;
            s->source = xcalloc(n1, sizeof(size_t)); s->target = xcalloc(n1, sizeof(size_t));
            for (size_t e = 0; e < n1; e++) { s->source[e] = src[e]; s->target[e] = tgt[e]; }
            free(src); free(tgt);
        } else {
            uint64_t e = rd_u(r), indegree = rd_u(r); tseed = rd_u(r);
            n_init = (size_t)rd_u(r);
            inits = xcalloc(n_init, sizeof *inits);
            for (size_t k = 0; k < n_init; k++) read_initializer(r, &inits[k]);
            if (topo == 1) TRY(build_fixed_total(s->scount, s->tcount, e, tseed, &s->source, &s->target, &s->n_edges));
            else {
                TRY(build_fixed_indegree(s->scount, s->tcount, indegree, tseed, &s->source, &s->target, &s->n_edges));
                if (s->n_edges != e) FAIL("fixed-indegree edge count mismatch");
            }
        }
        s->n_states = (size_t)rd_u(r);
        s->states = xcalloc(s->n_states, sizeof *s->states);
        for (size_t k = 0; k < s->n_states; k++) sa_read(r, &s->states[k]);
        s->n_tables = (size_t)rd_u(r);
        s->tables = xcalloc(s->n_tables, sizeof *s->tables);
        for (size_t k = 0; k < s->n_tables; k++) {
            if (rd_u(r) == 1) {
                uint64_t which = rd_u(r);
                s->tables[k] = xcalloc(s->n_edges, 8);
                TRY(materialize(&inits[which], s->n_edges, tseed, s->tables[k]));
            } else { size_t n; s->tables[k] = rd_f64s(r, &n); }
        }
        s->n_path = (size_t)rd_u(r);
        s->path = xcalloc(s->n_path, sizeof *s->path);
        for (size_t k = 0; k < s->n_path; k++) {
            Pathway *pw = &s->path[k];
            pw->is_pre = (int)rd_u(r);
            pw->event_index = (size_t)rd_u(r);
            if (rd_u(r) == 1) {
                Initializer init; read_initializer(r, &init);
                double dt = rd_f(r);
                double *values = xcalloc(s->n_edges, 8);
                TRY(materialize(&init, s->n_edges, tseed, values));
                pw->n_delay = s->n_edges; pw->delay = xcalloc(s->n_edges, sizeof(size_t));
                /* executor.rs:86-90: round-to-nearest tick quantisation of delays. */
                for (size_t e = 0; e < s->n_edges; e++) pw->delay[e] = (size_t)floor(values[e] / dt + 0.5);
                free(values);
            } else {
                uint64_t *d = rd_u64s(r, &pw->n_delay);
                pw->delay = xcalloc(pw->n_delay, sizeof(size_t));
                for (size_t e = 0; e < pw->n_delay; e++) pw->delay[e] = d[e];
                free(d);
            }
            size_t n_pending = (size_t)rd_u(r);
            uint64_t *pending = xcalloc(2 * n_pending, 8);
            for (size_t q = 0; q < 2 * n_pending; q++) pending[q] = rd_u(r);
            read_program(r, &pw->program, s->tables, m->seed);
            /* PathwayQueue::new (executor.rs:6185-6212). */
            const Population *endpoint = &m->pop[pw->is_pre ? s->spop : s->tpop];
            edge_csr(pw->is_pre ? s->source : s->target, s->n_edges, pw->is_pre ? s->scount : s->tcount,
                     &pw->offsets, &pw->edges);
            pw->uniform_delay = -1;
            size_t max_delay = 0;
            if (pw->n_delay) {
                int uniform = 1;
                for (size_t e = 0; e < pw->n_delay; e++) {
                    if (pw->delay[e] != pw->delay[0]) uniform = 0;
                    if (pw->delay[e] > max_delay) max_delay = pw->delay[e];
                }
                if (uniform) pw->uniform_delay = (int64_t)pw->delay[0];
            }
            pw->queue_len = max_delay + 1 < endpoint->steps ? max_delay + 1 : endpoint->steps;
            if (!pw->queue_len) FAIL("pathway queue has no slots");
            pw->queue = xcalloc(pw->queue_len, sizeof(VecZ));
            for (size_t q = 0; q < n_pending; q++) vz_push(&pw->queue[pending[2 * q] % pw->queue_len], pending[2 * q + 1]);
            free(pending);
        }
        s->n_code = (size_t)rd_u(r);
        s->codes = xcalloc(s->n_code, sizeof *s->codes);
        for (size_t k = 0; k < s->n_code; k++) {
            SynCode *c = &s->codes[k];
            c->kind = rd_u(r);
            if (c->kind == 0) {
                c->pathway = rd_u(r);
                if (c->pathway >= s->n_path) FAIL("synapse code object names no pathway");
            } else if (c->kind == 1) {
                read_program(r, &c->program, s->tables, m->seed);
            } else if (c->kind == 2) {
                c->to_pre = rd_u(r); c->state = rd_u(r); c->result = rd_u(r);
                c->start = rd_u(r); c->count = rd_u(r);
                read_program(r, &c->program, s->tables, m->seed);
            } else FAIL("unknown synapse code object kind");
        }
        free(inits);
    }
    m->n_nodes = (size_t)rd_u(r);
    m->nodes = xcalloc(m->n_nodes, sizeof *m->nodes);
    for (size_t k = 0; k < m->n_nodes; k++) {
        Node *nd = &m->nodes[k];
        nd->op = rd_u(r); nd->owner_kind = rd_u(r); nd->owner = rd_u(r); nd->item = rd_u(r); nd->clock = rd_u(r);
    }
    if (r->p != r->end) FAIL("oracle blob has trailing bytes");
    return 0;
}

/* run_program_neurons / run_population_update (executor.rs:2114-2164). */
static int run_population_program(Program *prog, Population *p, double time, uint64_t tick, int commit_avail) {
    TRY(program_prepare(prog, time, tick));
    for (size_t start = 0; start < p->count; start += LANES) {
        size_t len = p->count - start < LANES ? p->count - start : LANES;
        Batch b = batch_neurons(start, len);
        TRY(program_run(prog, p->states, p->states, p->states, NULL, p->has_refr ? &p->refr : NULL, &b));
        commit_neurons(prog, p->states, start, len);
        if (commit_avail && p->has_refr) commit_available(prog, &p->refr, start, len);
    }
    return 0;
}

/* emit_threshold (executor.rs:2949-3006). */
static int emit_threshold(Model *m, Population *p, Program *th, size_t event, int is_spike, double time) {
    VecZ *fired = &p->fired[event];
    fired->n = 0;
    TRY(program_prepare(th, time, p->tick));
    if (th->condition < 0) FAIL("missing threshold condition");
    for (size_t start = 0; start < p->count; start += LANES) {
        size_t len = p->count - start < LANES ? p->count - start : LANES;
        Batch b = batch_neurons(start, len);
        TRY(program_run(th, p->states, p->states, p->states, NULL, p->has_refr ? &p->refr : NULL, &b));
        for (size_t l = 0; l < len; l++) {
            size_t neuron = start + l;
            if (th->reg[th->condition][l] != 0.0 && (!is_spike || !p->has_refr || p->refr.not_refractory[neuron])) {
                vz_push(fired, neuron);
                if (is_spike && p->has_refr) { p->refr.lastspike[neuron] = time; p->refr.not_refractory[neuron] = 0; }
            }
        }
    }
    if (p->tick >= p->end_tick - p->window_steps) {
        if (!m->lift_budget && p->history[event].n / 2 + fired->n > 10000000) FAIL("event stream recording budget exceeded");
        for (size_t k = 0; k < fired->n; k++) { vz_push(&p->history[event], p->tick); vz_push(&p->history[event], fired->v[k]); }
    }
    return 0;
}

/* emit_spike_generator (executor.rs:3008-3036): the scheduled neurons of this tick, in
 * schedule order (ascending), after skipping entries before it. */
static int emit_spike_generator(Model *m, Population *p) {
    VecZ *fired = &p->fired[p->spike_event];
    fired->n = 0;
    while (p->gen_cursor < p->n_gen && p->gen_ticks[p->gen_cursor] < p->tick) p->gen_cursor++;
    while (p->gen_cursor < p->n_gen && p->gen_ticks[p->gen_cursor] == p->tick) {
        vz_push(fired, p->gen_neurons[p->gen_cursor]);
        p->gen_cursor++;
    }
    if (p->tick >= p->end_tick - p->window_steps) {
        if (!m->lift_budget && p->history[p->spike_event].n / 2 + fired->n > 10000000)
            FAIL("event stream recording budget exceeded");
        for (size_t k = 0; k < fired->n; k++) {
            vz_push(&p->history[p->spike_event], p->tick);
            vz_push(&p->history[p->spike_event], fired->v[k]);
        }
    }
    return 0;
}

/* deliver_event (executor.rs:2166-2251): one single-lane program run per edge. */
static int deliver_event(Model *m, Synapse *s, Program *prog, size_t source, size_t target, size_t edge) {
    Population *sp = &m->pop[s->spop], *tp = &m->pop[s->tpop];
    Batch b = { 0, 1, source, target, source + s->sstart, target + s->tstart, edge };
    TRY(program_run(prog, tp->states, sp->states, tp->states, s->states, tp->has_refr ? &tp->refr : NULL, &b));
    commit_event(prog, sp->states, tp->states, s->states, b.source_state, b.target_state, edge);
    return 0;
}

/* run_synapse_program (executor.rs:2513-2546): the clock-driven state update over every edge
 * in edge order, each edge's synapse states committed before the next. */
static int run_synapse_update(Model *m, Synapse *s, Program *prog, double time, size_t tick) {
    Population *sp = &m->pop[s->spop], *tp = &m->pop[s->tpop];
    TRY(program_prepare(prog, time, tick));
    for (size_t e = 0; e < s->n_edges; e++) {
        Batch b = { 0, 1, s->source[e], s->target[e], s->source[e] + s->sstart, s->target[e] + s->tstart, e };
        TRY(program_run(prog, tp->states, sp->states, tp->states, s->states, tp->has_refr ? &tp->refr : NULL, &b));
        for (size_t k = 0; k < prog->nw; k++)
            if (prog->w[k].kind == W_SYN) sa_set(&s->states[prog->w[k].index], e, prog->reg[prog->w[k].reg][0]);
    }
    return 0;
}

/* run_summed_program (executor.rs:2548-2597): the endpoint range of the target state set to
 * zero, then every edge's `_synaptic_var` added in edge order (add_f64, executor.rs:517-523: an
 * f32 state rounds after each addition). */
static int run_summed(Model *m, Synapse *s, SynCode *c, double time) {
    Population *sp = &m->pop[s->spop], *tp = &m->pop[s->tpop];
    Population *dest = c->to_pre ? sp : tp;
    StateArray *state = &dest->states[c->state];
    for (size_t k = c->start; k < c->start + c->count; k++) sa_set(state, k, 0.0);
    TRY(program_prepare(&c->program, time, dest->tick));
    for (size_t e = 0; e < s->n_edges; e++) {
        Batch b = { 0, 1, s->source[e], s->target[e], s->source[e] + s->sstart, s->target[e] + s->tstart, e };
        TRY(program_run(&c->program, tp->states, sp->states, tp->states, s->states, tp->has_refr ? &tp->refr : NULL,
                        &b));
        const size_t at = c->to_pre ? b.source_state : b.target_state;
        const double v = c->program.reg[c->result][0];
        if (state->dtype == DT_F32) sa_set(state, at, (double)(float)(sa_get(state, at) + v));
        else sa_set(state, at, sa_get(state, at) + v);
    }
    return 0;
}

/* run_pathway (executor.rs:2292-2382). */
static int run_pathway(Model *m, Synapse *s, Pathway *pw, double time) {
    size_t endpoint_pop = pw->is_pre ? s->spop : s->tpop;
    size_t start = pw->is_pre ? s->sstart : s->tstart, count = pw->is_pre ? s->scount : s->tcount;
    Population *ep = &m->pop[endpoint_pop];
    size_t tick = ep->tick, end_tick = ep->end_tick;
    pw->active.n = 0;
    VecZ *fired = &ep->fired[pw->event_index];
    for (size_t k = 0; k < fired->n; k++)
        if (fired->v[k] >= start && fired->v[k] < start + count) vz_push(&pw->active, fired->v[k] - start);
    if (pw->uniform_delay >= 0) {
        size_t delivery = tick + (size_t)pw->uniform_delay;
        if (delivery < end_tick)
            for (size_t k = 0; k < pw->active.n; k++) vz_push(&pw->queue[delivery % pw->queue_len], pw->active.v[k]);
    } else {
        for (size_t k = 0; k < pw->active.n; k++) {
            size_t endpoint = pw->active.v[k];
            for (size_t q = pw->offsets[endpoint]; q < pw->offsets[endpoint + 1]; q++) {
                size_t edge = pw->edges[q];
                size_t delivery = tick + pw->delay[edge];
                if (delivery < end_tick) vz_push(&pw->queue[delivery % pw->queue_len], edge);
            }
        }
    }
    VecZ *pending = &pw->queue[tick % pw->queue_len];
    TRY(program_prepare(&pw->program, time, tick));
    if (pw->uniform_delay >= 0) {
        for (size_t k = 0; k < pending->n; k++) {
            size_t endpoint = pending->v[k];
            for (size_t q = pw->offsets[endpoint]; q < pw->offsets[endpoint + 1]; q++) {
                size_t edge = pw->edges[q];
                TRY(deliver_event(m, s, &pw->program, s->source[edge], s->target[edge], edge));
                pw->delivered++;
            }
        }
    } else {
        for (size_t k = 0; k < pending->n; k++) {
            size_t edge = pending->v[k];
            TRY(deliver_event(m, s, &pw->program, s->source[edge], s->target[edge], edge));
            pw->delivered++;
        }
    }
    pending->n = 0;
    return 0;
}

/* record_states / record_spikes (executor.rs:3038-3087). */
static void record_states(Population *p) {
    if (p->tick < p->end_tick - p->window_steps) return;
    for (size_t r = 0; r < p->n_record; r++) {
        size_t neuron = p->record[r];
        for (size_t k = 0; k < p->n_mon; k++) {
            const MonitorValue *mv = &p->mon[k];
            double v = mv->kind == 0 ? sa_get(&p->states[mv->state], neuron) : mv->kind == 1 ? mv->scalar : mv->param[neuron];
            sa_push(&p->samples[k], v);
        }
    }
}
static void record_spikes(Population *p) {
    if (p->tick < p->end_tick - p->window_steps || p->spike_event < 0) return;
    VecZ *fired = &p->fired[p->spike_event];
    for (size_t k = 0; k < fired->n; k++) {
        p->counts[fired->v[k]]++;
        vz_push(&p->spikes, p->tick); vz_push(&p->spikes, fired->v[k]);
    }
}

/* record_events (executor.rs:3053-3080): the monitor's event list of this tick, with the
 * monitored values as stored at this schedule position. */
static int record_events(Model *m, Population *p, size_t k) {
    if (k >= p->n_emon) FAIL("scheduled EventMonitor has no runtime state");
    EventMonitor *em = &p->emon[k];
    const VecZ *fired = &p->fired[em->event];
    size_t samples = 0;
    for (size_t v = 0; v < em->n_vars; v++) samples += em->samples[v].len;
    if (!m->lift_budget && (em->events.n / 2 + fired->n > 10000000 || samples + fired->n * em->n_vars > 10000000))
        FAIL("EventMonitor recording budget exceeded");
    for (size_t f = 0; f < fired->n; f++) {
        size_t neuron = fired->v[f];
        vz_push(&em->events, p->tick); vz_push(&em->events, neuron);
        for (size_t v = 0; v < em->n_vars; v++) {
            const MonitorValue *mv = &em->vals[v];
            sa_push(&em->samples[v], mv->kind == 0 ? sa_get(&p->states[mv->state], neuron)
                                     : mv->kind == 1 ? mv->scalar : mv->param[neuron]);
        }
    }
    return 0;
}

/* Runtime::advance (executor.rs:3927-4361), schedule-dispatch branch. */
static int advance(Model *m, uint64_t max_ticks, uint64_t *ticks_run) {
    double epsilon = INFINITY;
    for (size_t c = 0; c < m->n_clocks; c++) epsilon = fmin(epsilon, m->clock_dt[c]);
    epsilon *= 1e-12;
    uint8_t *active = xcalloc(m->n_clocks, 1), *recorded = xcalloc(m->n_pop, 1);
    *ticks_run = 0;
    for (uint64_t iteration = 0; iteration < max_ticks; iteration++) {
        double time = INFINITY; int any = 0;
        for (size_t c = 0; c < m->n_clocks; c++)
            if (m->clock_tick[c] < m->clock_end[c]) { time = fmin(time, (double)m->clock_tick[c] * m->clock_dt[c]); any = 1; }
        if (!any) break;
        for (size_t c = 0; c < m->n_clocks; c++)
            active[c] = m->clock_tick[c] < m->clock_end[c]
                        && fabs((double)m->clock_tick[c] * m->clock_dt[c] - time) <= epsilon;
        memset(recorded, 0, m->n_pop);
        for (size_t k = 0; k < m->n_nodes; k++) {
            const Node *nd = &m->nodes[k];
            if (!active[nd->clock]) continue;
            size_t owner_clock = nd->owner_kind == 0 ? m->pop[nd->owner].clock : nd->clock;
            double now = (double)m->clock_tick[owner_clock] * m->clock_dt[owner_clock];
            if (nd->owner_kind == 0) {
                Population *p = &m->pop[nd->owner];
                if (nd->op == 1) { if (!recorded[nd->owner]) { record_states(p); recorded[nd->owner] = 1; } continue; }
                if (nd->op == 2) { record_spikes(p); continue; }
                if (nd->op == 3) { TRY(emit_spike_generator(m, p)); continue; }
                if (nd->op == 4) { TRY(record_events(m, p, (size_t)nd->item)); continue; }
                const int64_t *code = p->code[nd->item];
                Program *prog = &p->prog[code[0]][code[1]];
                switch (code[0]) {
                case PK_SUBEXPR: case PK_REGULAR:
                    TRY(run_population_program(prog, p, now, m->clock_tick[nd->clock], 0));
                    break;
                case PK_UPDATE:
                    if (p->has_refr && p->fixed_refr) {
                        /* executor.rs:4045-4058 */
                        for (size_t n = 0; n < p->count; n++) {
                            uint64_t ts; TRY(brian_timestep(now - p->refr.lastspike[n], p->dt, &ts));
                            p->refr.not_refractory[n] = ts >= p->period_ticks;
                        }
                    }
                    TRY(run_population_program(prog, p, now, m->clock_tick[nd->clock], 1));
                    break;
                case PK_THRESHOLD:
                    if (code[2] < 0) FAIL("scheduled threshold event is unknown");
                    TRY(emit_threshold(m, p, prog, (size_t)code[2], (int)code[3], now));
                    break;
                case PK_RESET: {
                    if (code[2] < 0) FAIL("scheduled reset event is unknown");
                    TRY(program_prepare(prog, now, m->clock_tick[nd->clock]));
                    VecZ *fired = &p->fired[code[2]];
                    for (size_t f = 0; f < fired->n; f++) {
                        Batch b = batch_neurons(fired->v[f], 1);
                        TRY(program_run(prog, p->states, p->states, p->states, NULL, p->has_refr ? &p->refr : NULL, &b));
                        commit_neurons(prog, p->states, fired->v[f], 1);
                    }
                    break;
                }
                default: FAIL("unsupported scheduled population operation");
                }
            } else {
                if (nd->op != 0) FAIL("unsupported synapse schedule operation");
                Synapse *s = &m->syn[nd->owner];
                if (nd->item >= s->n_code) FAIL("scheduled synapse code object is unknown");
                SynCode *c = &s->codes[nd->item];
                if (c->kind == 0) TRY(run_pathway(m, s, &s->path[c->pathway], now));
                else if (c->kind == 1) TRY(run_synapse_update(m, s, &c->program, now, m->clock_tick[nd->clock]));
                else TRY(run_summed(m, s, c, now));
            }
        }
        for (size_t pi = 0; pi < m->n_pop; pi++) {
            Population *p = &m->pop[pi];
            if (!active[p->clock]) continue;
            p->last_fired.n = 0;
            if (p->spike_event >= 0) {
                VecZ *fired = &p->fired[p->spike_event];
                for (size_t k = 0; k < fired->n; k++) vz_push(&p->last_fired, fired->v[k]);
            }
            p->tick = m->clock_tick[p->clock] + 1;
        }
        for (size_t c = 0; c < m->n_clocks; c++) m->clock_tick[c] += active[c];
        (*ticks_run)++;
    }
    free(active); free(recorded);
    return 0;
}

/* ----------------------------------------------------------------- dumps */
static void dump_state(VecB *o, const StateArray *a) { vb_put(o, a->data, a->len * dt_size(a->dtype)); }

/* write_dump (executor.rs:3147-3340), layout B2DMP001 version 3. */
static void write_results(const Model *m, VecB *o) {
    size_t size = 40;
    for (size_t pi = 0; pi < m->n_pop; pi++) {
        const Population *p = &m->pop[pi];
        size += 64 + p->spikes.n / 2 * 16 + p->count * 8 + p->last_fired.n * 8;
        for (size_t k = 0; k < p->n_mon; k++) size += p->samples[k].len * dt_size(p->samples[k].dtype);
        for (size_t k = 0; k < p->n_states; k++) size += p->states[k].len * dt_size(p->states[k].dtype);
        if (p->has_refr) size += p->count * 9;
    }
    size += 24;
    for (size_t si = 0; si < m->n_syn; si++) {
        size += 24;
        for (size_t k = 0; k < m->syn[si].n_states; k++) size += m->syn[si].states[k].len * dt_size(m->syn[si].states[k].dtype);
    }
    vb_put(o, "B2DMP001", 8);
    uint32_t version = 3, marker = 0x01020304;
    vb_put(o, &version, 4); vb_put(o, &marker, 4);
    vb_u64(o, m->n_pop); vb_u64(o, m->neuron_count); vb_u64(o, size);
    for (size_t pi = 0; pi < m->n_pop; pi++) {
        const Population *p = &m->pop[pi];
        vb_u64(o, p->count); vb_u64(o, p->steps); vb_u64(o, p->n_record); vb_u64(o, p->n_mon);
        vb_u64(o, p->n_states); vb_u64(o, p->spikes.n / 2); vb_u64(o, p->last_fired.n); vb_u64(o, (uint64_t)p->has_refr);
        for (size_t k = 0; k < p->n_mon; k++) dump_state(o, &p->samples[k]);
        for (size_t k = 0; k < p->spikes.n; k++) vb_u64(o, p->spikes.v[k]);
        for (size_t k = 0; k < p->count; k++) vb_u64(o, p->counts[k]);
        for (size_t k = 0; k < p->last_fired.n; k++) vb_u64(o, p->last_fired.v[k]);
        for (size_t k = 0; k < p->n_states; k++) dump_state(o, &p->states[k]);
        if (p->has_refr) {
            vb_put(o, p->refr.lastspike, p->count * 8);
            vb_put(o, p->refr.not_refractory, p->count);
        }
    }
    vb_u64(o, m->n_syn);
    for (size_t si = 0; si < m->n_syn; si++) {
        const Synapse *s = &m->syn[si];
        vb_u64(o, s->n_states); vb_u64(o, s->n_edges);
        for (size_t k = 0; k < s->n_states; k++) dump_state(o, &s->states[k]);
        uint64_t delivered = 0;
        for (size_t k = 0; k < s->n_path; k++) delivered += s->path[k].delivered;
        vb_u64(o, delivered);
    }
    double final_time = m->run_start + m->run_duration;
    vb_put(o, &final_time, 8);
    vb_put(o, "B2END001", 8);
}

/* write_event_monitor_dump (executor.rs:3342-3406), layout B2EVT001. */
static void write_events(const Model *m, VecB *o) {
    size_t streams = 0;
    for (size_t pi = 0; pi < m->n_pop; pi++) streams += m->pop[pi].n_events;
    vb_put(o, "B2EVT001", 8);
    vb_u64(o, streams);
    for (size_t pi = 0; pi < m->n_pop; pi++)
        for (size_t e = 0; e < m->pop[pi].n_events; e++) {
            const VecZ *h = &m->pop[pi].history[e];
            vb_u64(o, h->n / 2);
            for (size_t k = 0; k < h->n; k++) vb_u64(o, h->v[k]);
        }
    size_t monitors = 0;
    for (size_t pi = 0; pi < m->n_pop; pi++) monitors += m->pop[pi].n_emon;
    vb_u64(o, monitors);
    for (size_t pi = 0; pi < m->n_pop; pi++)
        for (size_t k = 0; k < m->pop[pi].n_emon; k++) {
            const EventMonitor *em = &m->pop[pi].emon[k];
            vb_u64(o, em->events.n / 2);
            vb_u64(o, em->n_vars);
            for (size_t q = 0; q < em->events.n; q++) vb_u64(o, em->events.v[q]);
            for (size_t v = 0; v < em->n_vars; v++) dump_state(o, &em->samples[v]);
        }
    vb_put(o, "B2EEND01", 8);
}

static void program_free(Program *p) {
    free(p->reg); free(p->b); free(p->scalar_random); free(p->broad); free(p->scalar); free(p->vector); free(p->w);
}
static void model_free(Model *m) {
    for (size_t pi = 0; pi < m->n_pop; pi++) {
        Population *p = &m->pop[pi];
        for (size_t k = 0; k < p->n_states; k++) free(p->states[k].data);
        free(p->states);
        if (p->has_refr) { free(p->refr.lastspike); free(p->refr.not_refractory); }
        for (size_t k = 0; k < p->n_mon; k++) { free(p->mon[k].param); free(p->samples[k].data); }
        free(p->mon); free(p->samples); free(p->record);
        for (size_t k = 0; k < p->n_tables; k++) free(p->tables[k]);
        free(p->tables);
        for (int kind = 0; kind < PK_COUNT; kind++) {
            for (size_t k = 0; k < p->n_prog[kind]; k++) program_free(&p->prog[kind][k]);
            free(p->prog[kind]);
        }
        free(p->code);
        for (size_t e = 0; p->fired && e < (p->n_events ? p->n_events : 1); e++) { free(p->fired[e].v); free(p->history[e].v); }
        free(p->fired); free(p->history); free(p->counts); free(p->last_fired.v); free(p->spikes.v);
        free(p->gen_ticks); free(p->gen_neurons);
        for (size_t k = 0; k < p->n_emon; k++) {
            EventMonitor *em = &p->emon[k];
            for (size_t v = 0; v < em->n_vars; v++) { free(em->vals[v].param); free(em->samples[v].data); }
            free(em->vals); free(em->samples); free(em->events.v);
        }
        free(p->emon);
    }
    free(m->pop);
    for (size_t si = 0; si < m->n_syn; si++) {
        Synapse *s = &m->syn[si];
        free(s->source); free(s->target);
        for (size_t k = 0; k < s->n_states; k++) free(s->states[k].data);
        free(s->states);
        for (size_t k = 0; k < s->n_tables; k++) free(s->tables[k]);
        free(s->tables);
        for (size_t k = 0; k < s->n_path; k++) {
            Pathway *pw = &s->path[k];
            program_free(&pw->program);
            free(pw->offsets); free(pw->edges); free(pw->delay); free(pw->active.v);
            for (size_t q = 0; pw->queue && q < pw->queue_len; q++) free(pw->queue[q].v);
            free(pw->queue);
        }
        for (size_t k = 0; s->codes && k < s->n_code; k++)
            if (s->codes[k].kind != 0) program_free(&s->codes[k].program);
        free(s->path); free(s->codes);
    }
    free(m->syn); free(m->nodes); free(m->clock_dt); free(m->clock_tick); free(m->clock_end);
}

/* -------------------------------------------------------------- public ABI */
int oracle_run(const uint8_t *blob, size_t len, int64_t max_ticks, OracleOutput *out, char *err, size_t cap) {
    memset(out, 0, sizeof *out);
    g_err[0] = 0;
    if (len < 8 || memcmp(blob, "ATLORC01", 8) != 0) { snprintf(err, cap, "bad oracle blob"); return 1; }
    Reader r = { blob + 8, blob + len };
    Model m; memset(&m, 0, sizeof m);
    if (load_model(&r, &m) != 0) { snprintf(err, cap, "%s", g_err); model_free(&m); return 1; }
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    uint64_t ticks = 0;
    int rc = advance(&m, max_ticks > 0 ? (uint64_t)max_ticks : UINT64_MAX, &ticks);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (rc != 0) { snprintf(err, cap, "%s", g_err); model_free(&m); return 2; }
    out->sim_seconds = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    out->ticks_run = ticks;
    VecB res = { 0 }, ev = { 0 };
    write_results(&m, &res);
    int has_events = 0;
    for (size_t pi = 0; pi < m.n_pop; pi++) if (m.pop[pi].n_events || m.pop[pi].n_emon) has_events = 1;
    if (has_events) write_events(&m, &ev);
    out->results = res.v; out->results_len = res.n;
    out->events = ev.v; out->events_len = ev.n; out->has_events = has_events;
    for (size_t pi = 0; pi < m.n_pop; pi++) out->spike_count += m.pop[pi].spikes.n / 2;
    for (size_t si = 0; si < m.n_syn; si++)
        for (size_t k = 0; k < m.syn[si].n_path; k++) out->synaptic_events += m.syn[si].path[k].delivered;
    model_free(&m);
    return 0;
}

void oracle_free(OracleOutput *out) {
    free(out->results); free(out->events);
    memset(out, 0, sizeof *out);
}

/* Known-answer hooks for the procedural generators (used by tests). */
int oracle_fixed_indegree(uint64_t n_src, uint64_t n_tgt, uint64_t indegree, uint64_t seed,
                          uint32_t *source_out, uint32_t *target_out) {
    size_t *s, *t, e;
    if (build_fixed_indegree(n_src, n_tgt, indegree, seed, &s, &t, &e) != 0) return 1;
    for (size_t k = 0; k < e; k++) { source_out[k] = (uint32_t)s[k]; target_out[k] = (uint32_t)t[k]; }
    free(s); free(t);
    return 0;
}
int oracle_fixed_total(uint64_t n_src, uint64_t n_tgt, uint64_t edges, uint64_t seed,
                       uint32_t *source_out, uint32_t *target_out) {
    size_t *s, *t, e;
    if (build_fixed_total(n_src, n_tgt, edges, seed, &s, &t, &e) != 0) return 1;
    for (size_t k = 0; k < e; k++) { source_out[k] = (uint32_t)s[k]; target_out[k] = (uint32_t)t[k]; }
    free(s); free(t);
    return 0;
}
int oracle_uniform(uint64_t count, uint64_t seed, uint64_t stream, double minimum, double maximum, double *out) {
    Initializer s = { 0, stream, minimum, maximum, 0, 0, 1, 1 };
    return materialize(&s, count, seed, out) != 0;
}
void oracle_set_shared_math(int enabled) { shared_math = enabled != 0; }

/* Test support: which = 0 exp, 1 expm1, 2 exprel, 3 log; writes the shared and the libm values. */
void oracle_math(int which, const double *x, size_t n, double *shared, double *libm) {
    for (size_t k = 0; k < n; k++) {
        const double v = x[k];
        if (which == 0) { shared[k] = atlas_exp(v); libm[k] = exp(v); }
        else if (which == 1) { shared[k] = atlas_expm1(v); libm[k] = expm1(v); }
        else if (which == 2) {
            shared[k] = atlas_exprel(v); libm[k] = fabs(v) < 1e-16 ? 1.0 : v > 717.0 ? INFINITY : expm1(v) / v;
        } else { shared[k] = atlas_log(v); libm[k] = log(v); }
    }
}

/* Per-edge initializer values (materialize_uniform / materialize_clipped_normal,
 * large_topology.rs:95-142): kind 0 uniform on [minimum, maximum), kind 1 clipped normal. */
int oracle_initializer(int kind, uint64_t count, uint64_t seed, uint64_t stream, double minimum, double maximum,
                       double mean, double std, int has_min, int has_max, double *out) {
    Initializer s = { kind, stream, minimum, maximum, mean, std, has_min, has_max };
    return materialize(&s, count, seed, out) != 0;
}

/* counter_normal (executor.rs:206-221) with the shared or the libm logarithm. */
double oracle_counter_normal(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index, int shared) {
    const int saved_shared = shared_math, saved_vector = in_vector;
    shared_math = shared != 0; in_vector = 1;
    const double value = counter_normal(seed, stream, tick, index);
    shared_math = saved_shared; in_vector = saved_vector;
    return value;
}

double oracle_counter_uniform(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index) {
    return counter_uniform(seed, stream, tick, index);
}

/* Test support for the binomial and Poisson draws, as vector code computes them (shared selects
 * the atlas_math.h logarithm and exponential, else the host libm). */
double oracle_counter_uniform_draw(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index, uint64_t draw) {
    return counter_uniform_draw(seed, stream, tick, index, draw);
}
double oracle_counter_binomial(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index, uint64_t n, double p,
                               int approximate, int shared) {
    const int saved_shared = shared_math, saved_vector = in_vector;
    shared_math = shared != 0; in_vector = 1;
    const double value = counter_binomial(seed, stream, tick, index, n, p, approximate);
    shared_math = saved_shared; in_vector = saved_vector;
    return value;
}
/* One inversion search on a chosen uniform, from the smaller tail of p (<= 0.5). */
double oracle_binomial_search(double u, uint64_t n, double probability, int shared) {
    const int saved_shared = shared_math, saved_vector = in_vector;
    shared_math = shared != 0; in_vector = 1;
    const double q = 1.0 - probability;
    const double qn = math_exp((double)n * math_log(q));
    const double bound = fmin((double)n, (double)n * probability + 10.0 * sqrt((double)n * probability * q + 1.0));
    const double value = binomial_search(u, n, probability, q, qn, bound);
    shared_math = saved_shared; in_vector = saved_vector;
    return value;
}
double oracle_counter_poisson(uint64_t seed, uint64_t stream, uint64_t tick, uint64_t index, double lambda,
                              int shared) {
    const int saved_shared = shared_math, saved_vector = in_vector;
    shared_math = shared != 0; in_vector = 1;
    const double value = counter_poisson(seed, stream, tick, index, lambda);
    shared_math = saved_shared; in_vector = saved_vector;
    return value;
}
double oracle_ptrs_trial(double u, double v, double lambda, int shared) {
    const int saved_shared = shared_math, saved_vector = in_vector;
    shared_math = shared != 0; in_vector = 1;
    const double value = ptrs_trial(u, v, lambda);
    shared_math = saved_shared; in_vector = saved_vector;
    return value;
}
