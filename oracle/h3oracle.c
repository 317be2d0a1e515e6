/* h3oracle.c - CPU restatement of the reference's per-token layer arithmetic (see h3oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker the GPU library is compared against, never part of the product path.
 * Build with -ffp-contract=off (oracle/Makefile): every rounding step below is the one written.
 */
#include "h3oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];
static int g_threads = 1;

static int fail(const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return -1;
}
const char* h3o_last_error(void) { return g_err; }

void h3o_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int h3o_get_threads(void) { return g_threads; }

/* ---- row-parallel driver: contiguous row chunks, one per thread (engine/h3-core/src/reference.rs:43-80) ---- */
typedef void (*row_fn)(void* ctx, int64_t r0, int64_t r1);
typedef struct { row_fn fn; void* ctx; int64_t r0, r1; } job;
static void* run_job(void* p) {
    job* j = (job*) p;
    j->fn(j->ctx, j->r0, j->r1);
    return NULL;
}
static void parallel_rows(int64_t M, row_fn fn, void* ctx) {
    int t = g_threads > 256 ? 256 : g_threads;
    if (t > M) t = (int) (M > 0 ? M : 1);
    if (t <= 1) { fn(ctx, 0, M); return; }
    const int64_t per = (M + t - 1) / t;
    pthread_t th[256];
    job jobs[256];
    int made[256] = {0};
    for (int i = 0; i < t; ++i) {
        const int64_t a = (int64_t) i * per, b = a + per < M ? a + per : M;
        if (a >= b) break;
        jobs[i] = (job){fn, ctx, a, b};
        if (pthread_create(&th[i], NULL, run_job, &jobs[i]) == 0) made[i] = 1;
        else fn(ctx, a, b);                                  /* no thread: do the chunk here */
    }
    for (int i = 0; i < t; ++i)
        if (made[i]) pthread_join(th[i], NULL);
}

/* ---- element types: dtype.rs:53-121 (bf16 narrowing also kernels/h3sycl.cpp:42-49) ---- */
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float h3o_bf16_to_f32(uint16_t b) { return bitsf((uint32_t) b << 16); }                       /* dtype.rs:54-56 */
uint16_t h3o_f32_to_bf16(float f) {                                                            /* dtype.rs:59-66 */
    uint32_t u = fbits(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t) (u >> 16);   /* inf / nan: truncate */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}
float h3o_f16_to_f32(uint16_t h) {                                                             /* dtype.rs:69-85 */
    const uint32_t sign = (uint32_t) (h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0 && man == 0) bits = sign;
    else if (exp == 0) {
        uint32_t m = man, shift = 0;
        while (!(m & 0x400)) { m <<= 1; ++shift; }          /* leading_zeros(man) - 21 of a u32 */
        bits = sign | ((113 - shift) << 23) | ((m & 0x3ff) << 13);
    } else if (exp == 31) bits = sign | 0x7f800000u | (man << 13);
    else bits = sign | ((exp + 112) << 23) | (man << 13);
    return bitsf(bits);
}
uint16_t h3o_f32_to_f16(float f) {                                                             /* dtype.rs:88-121 */
    const uint32_t u = fbits(f);
    const uint16_t sign = (uint16_t) ((u >> 16) & 0x8000);
    const int exp = (int) ((u >> 23) & 0xff);
    const uint32_t man = u & 0x7fffff;
    if (exp == 0xff) return sign | 0x7c00 | (man ? 0x200 : 0);
    const int e = exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t m = man | 0x800000, shift = (uint32_t) (14 - e), half = 1u << (shift - 1);
        const uint32_t rest = m & ((1u << shift) - 1);
        uint32_t hv = m >> shift;
        if (rest > half || (rest == half && (hv & 1))) hv += 1;
        return sign | (uint16_t) hv;
    }
    uint32_t hv = ((uint32_t) e << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fff;
    if (rest > 0x1000 || (rest == 0x1000 && (hv & 1))) hv += 1;
    return sign | (uint16_t) hv;
}
float h3o_load(const void* p, int dt, int64_t i) {                                             /* h3sycl.cpp:50-56 */
    switch (dt) {
        case H3O_F16: return h3o_f16_to_f32(((const uint16_t*) p)[i]);
        case H3O_BF16: return h3o_bf16_to_f32(((const uint16_t*) p)[i]);
        default: return ((const float*) p)[i];
    }
}
void h3o_store(void* p, int dt, int64_t i, float v) {                                          /* h3sycl.cpp:57-63 */
    switch (dt) {
        case H3O_F16: ((uint16_t*) p)[i] = h3o_f32_to_f16(v); break;
        case H3O_BF16: ((uint16_t*) p)[i] = h3o_f32_to_bf16(v); break;
        default: ((float*) p)[i] = v;
    }
}
float h3o_round_to(float v, int dt) {
    switch (dt) {
        case H3O_F16: return h3o_f16_to_f32(h3o_f32_to_f16(v));
        case H3O_BF16: return h3o_bf16_to_f32(h3o_f32_to_bf16(v));
        default: return v;
    }
}
static int vec_of(int dt) { return dt == H3O_F32 ? 4 : 8; }   /* 16 bytes of the type: the kernels' load width */
static int dt_ok(int dt) { return dt == H3O_F32 || dt == H3O_F16 || dt == H3O_BF16; }

/* ---- seeded inputs: engine/h3-core/src/rng.rs:9-43 ---- */
void h3o_rng_new(h3o_rng* r, uint64_t seed) {                                                  /* rng.rs:9-20 */
    uint64_t z = seed;
    for (int i = 0; i < 4; ++i) {
        z += 0x9e3779b97f4a7c15ull;
        uint64_t x = z;
        x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
        x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
        r->s[i] = x ^ (x >> 31);
    }
}
void h3o_rng_from_state(h3o_rng* r, const uint64_t s[4]) { memcpy(r->s, s, sizeof r->s); }
static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
uint64_t h3o_rng_next_u64(h3o_rng* r) {                                                        /* rng.rs:22-31 */
    uint64_t* s = r->s;
    const uint64_t res = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return res;
}
float h3o_rng_uniform(h3o_rng* r) {                                                            /* rng.rs:34-36 */
    return (float) (h3o_rng_next_u64(r) >> 40) / (float) (1ull << 24);
}
float h3o_rng_normal(h3o_rng* r) {                                                             /* rng.rs:39-43 */
    float u = h3o_rng_uniform(r);
    u = u > 1e-7f ? u : 1e-7f;
    const float v = h3o_rng_uniform(r);
    const float tau = 6.28318530717958647692f;
    return sqrtf(-2.0f * logf(u)) * cosf(tau * v);
}
void h3o_fill_normal(uint64_t seed, float scale, int64_t n, void* out, int dt) {
    h3o_rng r;
    h3o_rng_new(&r, seed);
    for (int64_t i = 0; i < n; ++i) h3o_store(out, dt, i, h3o_rng_normal(&r) * scale);
}
void h3o_fill_uniform(uint64_t seed, float lo, float hi, int64_t n, float* out) {
    h3o_rng r;
    h3o_rng_new(&r, seed);
    for (int64_t i = 0; i < n; ++i) out[i] = lo + (hi - lo) * h3o_rng_uniform(&r);
}
void h3o_choose(uint64_t seed, int64_t n, int64_t k, int64_t* out) {
    h3o_rng r;
    h3o_rng_new(&r, seed);
    int64_t* idx = (int64_t*) malloc((size_t) n * sizeof(int64_t));
    for (int64_t i = 0; i < n; ++i) idx[i] = i;
    for (int64_t i = 0; i < k && i < n; ++i) {
        const int64_t j = i + (int64_t) (h3o_rng_next_u64(&r) % (uint64_t) (n - i));
        const int64_t t = idx[i]; idx[i] = idx[j]; idx[j] = t;
        out[i] = idx[i];
    }
    free(idx);
}

/* ---- canonical reduction ----
 * L lane partials, L a power of two up to 512. Up to 64 lanes (one wavefront): the xor butterfly with offsets
 * L/2, ..., 1. Beyond: that butterfly inside each group of 64 lanes first, then the same butterfly over the L/64
 * group sums (offsets L/128, ..., 1). */
static float butterfly(float* p, int L) {
    float tmp[512];
    for (int off = L / 2; off >= 1; off /= 2) {
        for (int l = 0; l < L; ++l) tmp[l] = p[l] + p[l ^ off];
        memcpy(p, tmp, (size_t) L * sizeof(float));
    }
    return p[0];
}
static float canon_combine(float* p, int L) {
    if (L <= 64) return butterfly(p, L);
    float w[8];
    for (int g = 0; g < L / 64; ++g) w[g] = butterfly(p + 64 * g, 64);
    return butterfly(w, L / 64);
}
float h3o_canon_sum(const float* x, int64_t n, int V, int L, int kind, float mean) {
    float p[512];
    for (int l = 0; l < L; ++l) p[l] = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const int l = (int) ((i / V) % L);
        const float v = x[i];
        if (kind == H3O_SUM) p[l] = p[l] + v;
        else if (kind == H3O_SUMSQ) p[l] = fmaf(v, v, p[l]);
        else { const float d = v - mean; p[l] = fmaf(d, d, p[l]); }
    }
    return canon_combine(p, L);
}
/* lanes per row of n values in 16-byte chunks of V: 64 below 256 chunks, 256 up to 1024, 512 up to 2048 */
int h3o_row_lanes(int64_t n, int V) {
    const int64_t nch = n / V;
    return nch < 256 ? 64 : nch <= 1024 ? 256 : 512;
}

/* 1 / sqrt(mean + eps), each step correctly rounded (the reference's sycl::rsqrt, h3sycl.cpp:779, 1264) */
static inline float inv_root(float sum, int64_t n, float eps) { return 1.0f / sqrtf(sum / (float) n + eps); }

/* ---- rms_norm_mod: kernels/h3sycl.cpp:766-810 (per element h3sycl.cpp:752-758, 802-806) ---- */
typedef struct {
    const void* x; int x_dt; int64_t C; const float* w; float eps; const int32_t* rows; const float* scale;
    const float* shift; void* out; int out_dt;
} rmsn_ctx;
static void rmsn_rows(void* p, int64_t r0, int64_t r1) {
    const rmsn_ctx* c = (const rmsn_ctx*) p;
    const int64_t C = c->C;
    float* row = (float*) malloc((size_t) C * sizeof(float));
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t i = 0; i < C; ++i) row[i] = h3o_load(c->x, c->x_dt, r * C + i);
        const float inv = inv_root(h3o_canon_sum(row, C, vec_of(c->x_dt), h3o_row_lanes(C, vec_of(c->x_dt)), H3O_SUMSQ, 0.0f), C, c->eps);
        for (int64_t i = 0; i < C; ++i) {
            float v = row[i] * inv * c->w[i];
            if (c->rows) {
                const int64_t m = (int64_t) c->rows[r] * C + i;
                v = v * (1.0f + c->scale[m]) + c->shift[m];
            }
            h3o_store(c->out, c->out_dt, r * C + i, v);
        }
    }
    free(row);
}
int h3o_rms_norm_mod(const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps, const int32_t* rows,
                     const float* scale, const float* shift, void* out, int out_dt) {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(out_dt)) return fail("rms_norm_mod: unknown element type");
    const int mod = rows && scale && shift;
    rmsn_ctx c = {x, x_dt, C, weight, eps, mod ? rows : NULL, scale, shift, out, out_dt};
    parallel_rows(M, rmsn_rows, &c);
    return 0;
}

/* ---- layer_norm: kernels/h3sycl.cpp:1248-1274 (two passes over the row, then (x - mean) * inv, * w, + b) ---- */
typedef struct {
    const void* x; int x_dt; int64_t C; const float* w; const float* b; float eps; void* out; int out_dt;
} ln_ctx;
static void ln_stats(const float* row, int64_t C, int V, float eps, float* mean, float* inv) {
    const int L = h3o_row_lanes(C, V);
    *mean = h3o_canon_sum(row, C, V, L, H3O_SUM, 0.0f) / (float) C;
    *inv = inv_root(h3o_canon_sum(row, C, V, L, H3O_SUMSQ_DIFF, *mean), C, eps);
}
static void ln_rows(void* p, int64_t r0, int64_t r1) {
    const ln_ctx* c = (const ln_ctx*) p;
    const int64_t C = c->C;
    float* row = (float*) malloc((size_t) C * sizeof(float));
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t i = 0; i < C; ++i) row[i] = h3o_load(c->x, c->x_dt, r * C + i);
        float mean, inv;
        ln_stats(row, C, vec_of(c->x_dt), c->eps, &mean, &inv);
        for (int64_t i = 0; i < C; ++i) {
            float v = (row[i] - mean) * inv;
            if (c->w) v *= c->w[i];
            if (c->b) v += c->b[i];
            h3o_store(c->out, c->out_dt, r * C + i, v);
        }
    }
    free(row);
}
int h3o_layer_norm(const void* x, int x_dt, int64_t M, int64_t C, const float* weight, const float* bias, float eps,
                   void* out, int out_dt) {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(out_dt)) return fail("layer_norm: unknown element type");
    ln_ctx c = {x, x_dt, C, weight, bias, eps, out, out_dt};
    parallel_rows(M, ln_rows, &c);
    return 0;
}

/* ---- rms_rope: kernels/h3sycl.cpp:1276-1376 ----
 * Canonical per-head order: the head's D features are D / V 16-byte chunks (V the elements of a vector), chunk l
 * summed in order into partial l, the partials padded with zeros to CL = pow2ceil(D / V) and combined by the xor
 * butterfly: h3o_canon_sum over CL lanes. Then each pair (j, half + j), half = rot_dim / 2, rotates by the token's
 * (cos, sin) of j (h3sycl.cpp:1325-1331), and the features from rot_dim on are only normalized (h3sycl.cpp:1345). */
static int pow2ceil(int n) { int p = 1; while (p < n) p *= 2; return p; }
typedef struct {
    void* x; int x_dt; int64_t H, D, stride; const float* w; float eps; const float* cs; int rot;
} rope_ctx;
static void rope_rows(void* p, int64_t r0, int64_t r1) {
    const rope_ctx* c = (const rope_ctx*) p;
    const int64_t D = c->D, half = c->rot / 2;
    const int V = vec_of(c->x_dt);
    /* the head's sum of squares: the canonical sum over pow2ceil(D / V) lanes, one 16-byte chunk of the head a lane
     * (the reference's order, a sequential s += v * v, h3sycl.cpp:1296-1300, is left to its device: not restated) */
    const int CL = pow2ceil((int) (D / V));
    float* v = (float*) malloc((size_t) D * sizeof(float));
    for (int64_t m = r0; m < r1; ++m)
        for (int64_t h = 0; h < c->H; ++h) {
            const int64_t base = m * c->stride + h * D;
            for (int64_t i = 0; i < D; ++i) v[i] = h3o_load(c->x, c->x_dt, base + i);
            const float inv = inv_root(h3o_canon_sum(v, D, V, CL, H3O_SUMSQ, 0.0f), D, c->eps);
            for (int64_t j = 0; j < half; ++j) {
                const float a = v[j] * inv * c->w[j], b = v[half + j] * inv * c->w[half + j];
                const int64_t t = m * half + j;
                const float co = c->cs[2 * t], si = c->cs[2 * t + 1];
                h3o_store(c->x, c->x_dt, base + j, a * co - b * si);
                h3o_store(c->x, c->x_dt, base + half + j, b * co + a * si);
            }
            for (int64_t i = c->rot; i < D; ++i) h3o_store(c->x, c->x_dt, base + i, v[i] * inv * c->w[i]);
        }
    free(v);
}
int h3o_rms_rope(void* x, int x_dt, int64_t M, int64_t H, int64_t D, int64_t stride, const float* weight, float eps,
                 const float* cs, int rot_dim) {
    if (M <= 0 || H <= 0 || D <= 0) return 0;
    if (rot_dim < 0 || rot_dim > D || rot_dim % 2 != 0 || (D - rot_dim) % 2 != 0)
        return fail("rms_rope: rot_dim must be even, at most D, and leave an even remainder");
    if (stride < H * D) return fail("rms_rope: the row stride is shorter than a row");
    if (!dt_ok(x_dt)) return fail("rms_rope: unknown element type");
    const int V = vec_of(x_dt);
    if (D % V != 0 || D / V > 64) return fail("rms_rope: a head of whole 16-byte vectors, at most 64 of them");
    rope_ctx c = {x, x_dt, H, D, stride, weight, eps, cs, rot_dim};
    parallel_rows(M, rope_rows, &c);
    return 0;
}

/* ---- activations: SiLU h3sycl.cpp:1395, 1416; GELU-tanh engine/h3-core/src/audio.rs:440 ---- */
float h3o_act(float v, int act) {
    if (act == H3O_ACT_SILU) return v / (1.0f + expf(-v));
    if (act == H3O_ACT_GELU_TANH) {
        const float k = sqrtf(2.0f / 3.14159265358979323846f);
        return 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v * v * v)));
    }
    return v;
}
void h3o_act_n(const float* v, int64_t n, int act, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = h3o_act(v[i], act);
}

/* ---- swiglu: kernels/h3sycl.cpp:1378-1419 ---- */
int h3o_swiglu(const void* x, int x_dt, int64_t M, int64_t C, void* out, int out_dt) {
    if (M <= 0 || C <= 0) return 0;
    for (int64_t r = 0; r < M; ++r)
        for (int64_t i = 0; i < C; ++i) {
            const float g = h3o_load(x, x_dt, r * 2 * C + i), u = h3o_load(x, x_dt, r * 2 * C + C + i);
            h3o_store(out, out_dt, r * C + i, g / (1.0f + expf(-g)) * u);
        }
    return 0;
}

/* ---- gate_add: kernels/h3sycl.cpp:1421-1431 ---- */
int h3o_gate_add(void* x, int x_dt, int64_t M, int64_t C, const void* other, int other_dt, const int32_t* rows,
                 const float* gate) {
    if (M <= 0 || C <= 0) return 0;
    if (gate && !rows) return fail("gate_add: a gate needs the row table");
    for (int64_t r = 0; r < M; ++r)
        for (int64_t i = 0; i < C; ++i) {
            const int64_t p = r * C + i;
            const float g = gate ? gate[(int64_t) rows[r] * C + i] : 1.0f;
            h3o_store(x, x_dt, p, h3o_load(x, x_dt, p) + h3o_load(other, other_dt, p) * g);
        }
    return 0;
}

/* ---- rotations ---- */
/* regular: one base-4 digit at a time, low digit first (kernels/h3sycl.cpp:433-456). For the four values x0..x3
 * that differ only in that digit, y_a = t - 2 x_(3-a), with t formed as the reference's group-of-256 kernel forms
 * it: its work-item holds 16 consecutive features, so the digits of stride 1 and 4 are summed in registers left to
 * right, t = ((x0 + x1) + x2) + x3 (h3sycl.cpp:440), and the digits of stride 16 and 64 across the lanes, pairwise,
 * t = (x0 + x1) + (x2 + x3) (h3sycl.cpp:452-453). Then * 1/sqrt(g), a power of two (h3sycl.cpp:456). The smaller
 * groups (4, 16, 64) take the same rule by stride. Every digit forms t - 2 x with one rounding, fmaf(-2, x, t): the
 * reference's t - 2.0f * x (h3sycl.cpp:441, 454), which icpx -O3 contracts into that fma under its default
 * floating-point model (container/build-inside.sh:12); 2 x is exact for |x| < 2^127, so the two agree unless 2 x
 * overflows.
 * Sylvester: h = 1, 2, ..., g/2, (a, b) -> (a + b, a - b); then * fl(1/sqrt(g)). */
void h3o_rotate_group(float* y, int g, int kind) {
    if (kind == H3O_ROT_REGULAR) {
        for (int d = 1; d < g; d *= 4)
            for (int i = 0; i < g; ++i) {
                if ((i / d) % 4 != 0) continue;
                const float x0 = y[i], x1 = y[i + d], x2 = y[i + 2 * d], x3 = y[i + 3 * d];
                const float t = d < 16 ? ((x0 + x1) + x2) + x3 : (x0 + x1) + (x2 + x3);
                y[i] = fmaf(-2.0f, x3, t);
                y[i + d] = fmaf(-2.0f, x2, t);
                y[i + 2 * d] = fmaf(-2.0f, x1, t);
                y[i + 3 * d] = fmaf(-2.0f, x0, t);
            }
    } else if (kind == H3O_ROT_SYLVESTER) {
        for (int h = 1; h < g; h *= 2)
            for (int i = 0; i < g; ++i) {
                if (i & h) continue;
                const float a = y[i], b = y[i + h];
                y[i] = a + b;
                y[i + h] = a - b;
            }
    } else return;
    const float c = (float) (1.0 / sqrt((double) g));
    for (int i = 0; i < g; ++i) y[i] = y[i] * c;
}
void h3o_hadamard_regular(int g, float* h) {                                                   /* reference.rs:4-23 */
    static const int h4[4][4] = {{1, 1, 1, -1}, {1, 1, -1, 1}, {1, -1, 1, 1}, {-1, 1, 1, 1}};
    const float norm = 1.0f / sqrtf((float) g);
    for (int i = 0; i < g; ++i)
        for (int j = 0; j < g; ++j) {
            int a = i, b = j, s = 1, sign = 1;
            while (s < g) { sign *= h4[a % 4][b % 4]; a /= 4; b /= 4; s *= 4; }
            h[(int64_t) i * g + j] = (float) sign * norm;
        }
}
void h3o_hadamard_sylvester(int g, float* h) {
    const float norm = (float) (1.0 / sqrt((double) g));
    for (int i = 0; i < g; ++i)
        for (int j = 0; j < g; ++j) h[(int64_t) i * g + j] = (__builtin_popcount((unsigned) (i & j)) & 1) ? -norm : norm;
}

/* ---- quantizer: kernels/h3sycl.h:74-83; h3sycl.cpp:465-472, 556-573; reference.rs:68-70 ---- */
static void quantize_row(const float* y, int64_t K, int8_t* q, float* s) {
    float m = 0.0f;
    for (int64_t i = 0; i < K; ++i) m = fmaxf(m, fabsf(y[i]));
    const float sc = fmaxf(m / 127.0f, 1e-30f);
    *s = sc;
    for (int64_t i = 0; i < K; ++i) {
        float v = rintf(y[i] / sc);
        v = v < -128.0f ? -128.0f : v > 127.0f ? 127.0f : v;
        q[i] = (int8_t) v;
    }
}
void h3o_quantize_rows(const float* y, int64_t M, int64_t K, int8_t* q, float* s) {
    for (int64_t r = 0; r < M; ++r) quantize_row(y + r * K, K, q + r * K, s + r);
}

/* ---- int8 GEMM + dequant epilogue: kernels/h3sycl.cpp:576-629, reference.rs:72-76 ----
 * One weight scale: the row factor is fl(s_r * wscale[0]) (h3sycl.cpp:576), out = acc * factor. One per output:
 * out = (acc * s_r) * wscale[n] (the post-op chain h3sycl.cpp:588-602). Then + bias[n], then the activation. */
typedef struct {
    const int8_t* q; const float* s; int64_t K; const int8_t* w; int64_t N; const float* ws; int64_t nws;
    const float* bias; int act; void* out; int out_dt;
} gemm_ctx;
static void gemm_rows(void* p, int64_t r0, int64_t r1) {
    const gemm_ctx* c = (const gemm_ctx*) p;
    const int64_t K = c->K;
    for (int64_t r = r0; r < r1; ++r) {
        const int8_t* qr = c->q + r * K;
        const float sr = c->s[r];
        const float f1 = sr * c->ws[0];
        for (int64_t n = 0; n < c->N; ++n) {
            const int8_t* wr = c->w + n * K;
            int32_t acc = 0;
            for (int64_t k = 0; k < K; ++k) acc += (int32_t) qr[k] * (int32_t) wr[k];
            float v = c->nws == 1 ? (float) acc * f1 : (float) acc * sr * c->ws[n];
            if (c->bias) v = v + c->bias[n];
            v = h3o_act(v, c->act);
            h3o_store(c->out, c->out_dt, r * c->N + n, v);
        }
    }
}
int h3o_gemm_dequant(const int8_t* q, const float* s, int64_t M, int64_t K, const int8_t* w, int64_t N, const float* wscale,
                     int64_t n_wscale, const float* bias, int act, void* out, int out_dt) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (n_wscale != 1 && n_wscale != N) return fail("gemm_dequant: 1 or N weight scales");
    gemm_ctx c = {q, s, K, w, N, wscale, n_wscale, bias, act, out, out_dt};
    parallel_rows(M, gemm_rows, &c);
    return 0;
}

/* ---- int8_linear: kernels/h3sycl.h:74-85; h3sycl.cpp:633-652 ---- */
typedef struct { const void* x; int x_dt; int64_t K; int group; int8_t* q; float* s; } quant_ctx;
static void quant_rows(void* p, int64_t r0, int64_t r1) {
    const quant_ctx* c = (const quant_ctx*) p;
    float* y = (float*) malloc((size_t) c->K * sizeof(float));
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t i = 0; i < c->K; ++i) y[i] = h3o_load(c->x, c->x_dt, r * c->K + i);
        if (c->group > 0)
            for (int64_t g0 = 0; g0 < c->K; g0 += c->group) h3o_rotate_group(y + g0, c->group, H3O_ROT_REGULAR);
        quantize_row(y, c->K, c->q + r * c->K, c->s + r);
    }
    free(y);
}
static int is_pow4(int g) { return g > 0 && (g & (g - 1)) == 0 && (__builtin_ctz((unsigned) g) % 2) == 0; }
int h3o_int8_linear(const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N, const float* wscale,
                    int64_t n_wscale, const float* bias, void* out, int out_dt, int group) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (group > 0 && (group > 256 || K % group != 0 || !is_pow4(group)))
        return fail("int8_linear: the ConvRot group must be a power of 4, at most 256, dividing K");
    int8_t* q = (int8_t*) malloc((size_t) (M * K));
    float* s = (float*) malloc((size_t) M * sizeof(float));
    quant_ctx qc = {x, x_dt, K, group, q, s};
    parallel_rows(M, quant_rows, &qc);
    const int rc = h3o_gemm_dequant(q, s, M, K, w, N, wscale, n_wscale, bias, H3O_ACT_NONE, out, out_dt);
    free(q);
    free(s);
    return rc;
}

/* ---- fused chains ---- */
typedef struct {
    const void* x; int x_dt; int64_t C; const float* w; float eps; const int32_t* rows; const void* scale;
    const void* shift; int tab_dt; int h_dt; int rot; int group; int8_t* q; float* s;
} nq_ctx;
static void nq_rows(void* p, int64_t r0, int64_t r1) {
    const nq_ctx* c = (const nq_ctx*) p;
    const int64_t C = c->C;
    float* y = (float*) malloc((size_t) C * sizeof(float));
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t i = 0; i < C; ++i) y[i] = h3o_load(c->x, c->x_dt, r * C + i);
        const float inv = inv_root(h3o_canon_sum(y, C, vec_of(c->x_dt), h3o_row_lanes(C, vec_of(c->x_dt)), H3O_SUMSQ, 0.0f), C, c->eps);
        const int64_t tr = c->rows ? c->rows[r] : 0;
        for (int64_t i = 0; i < C; ++i) {
            float v = y[i] * inv;
            if (c->w) v = v * c->w[i];
            if (c->scale && c->shift) {
                const float sc = h3o_load(c->scale, c->tab_dt, tr * C + i), sh = h3o_load(c->shift, c->tab_dt, tr * C + i);
                v = v * (1.0f + sc) + sh;
            }
            y[i] = h3o_round_to(v, c->h_dt);
        }
        if (c->rot != H3O_ROT_NONE)
            for (int64_t g0 = 0; g0 < C; g0 += c->group) h3o_rotate_group(y + g0, c->group, c->rot);
        quantize_row(y, C, c->q + r * C, c->s + r);
    }
    free(y);
}
int h3o_norm_quant(const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps, const int32_t* rows,
                   const void* scale, const void* shift, int tab_dt, int h_dt, int rot, int group, int8_t* q, float* s) {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(h_dt) || !dt_ok(tab_dt)) return fail("norm_quant: unknown element type");
    if (rot == H3O_ROT_REGULAR && (!is_pow4(group) || C % group != 0)) return fail("norm_quant: regular rotation needs g = 4^k dividing C");
    if (rot == H3O_ROT_SYLVESTER && (group < 2 || (group & (group - 1)) != 0 || C % group != 0))
        return fail("norm_quant: Sylvester rotation needs g = 2^k dividing C");
    nq_ctx c = {x, x_dt, C, weight, eps, rows, scale, shift, tab_dt, h_dt, rot, group, q, s};
    parallel_rows(M, nq_rows, &c);
    return 0;
}

/* ---- swiglu into the MLP's act scratch, then fc2's quantizer (dit.rs:363-364; h3sycl.cpp:1378-1419, 404-474);
 * with swiglu == 0 the quantizer alone on x (rows of C): h3s_int8_linear's quantizer with any rotation kind ---- */
typedef struct {
    const void* x; int x_dt; int64_t C; int h_dt; int rot; int group; int swiglu; int8_t* q; float* s;
} sq_ctx;
static void sq_rows(void* p, int64_t r0, int64_t r1) {
    const sq_ctx* c = (const sq_ctx*) p;
    const int64_t C = c->C;
    float* y = (float*) malloc((size_t) C * sizeof(float));
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t i = 0; i < C; ++i) {
            if (c->swiglu) {
                const float g = h3o_load(c->x, c->x_dt, r * 2 * C + i), u = h3o_load(c->x, c->x_dt, r * 2 * C + C + i);
                y[i] = h3o_round_to(g / (1.0f + expf(-g)) * u, c->h_dt);        /* h3sycl.cpp:1396, 1416 */
            } else {
                y[i] = h3o_load(c->x, c->x_dt, r * C + i);
            }
        }
        if (c->rot != H3O_ROT_NONE)
            for (int64_t g0 = 0; g0 < C; g0 += c->group) h3o_rotate_group(y + g0, c->group, c->rot);
        quantize_row(y, C, c->q + r * C, c->s + r);
    }
    free(y);
}
static int sq_run(const void* x, int x_dt, int64_t M, int64_t C, int h_dt, int rot, int group, int swiglu, int8_t* q, float* s) {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(h_dt)) return fail("swiglu_quant: unknown element type");
    if (rot == H3O_ROT_REGULAR && (!is_pow4(group) || C % group != 0)) return fail("swiglu_quant: regular rotation needs g = 4^k dividing C");
    if (rot == H3O_ROT_SYLVESTER && (group < 2 || (group & (group - 1)) != 0 || C % group != 0))
        return fail("swiglu_quant: Sylvester rotation needs g = 2^k dividing C");
    sq_ctx c = {x, x_dt, C, h_dt, rot, group, swiglu, q, s};
    parallel_rows(M, sq_rows, &c);
    return 0;
}
int h3o_swiglu_quant(const void* x, int x_dt, int64_t M, int64_t C, int h_dt, int rot, int group, int8_t* q, float* s) {
    return sq_run(x, x_dt, M, C, h_dt, rot, group, 1, q, s);
}
int h3o_quantize_act(const void* x, int x_dt, int64_t M, int64_t C, int rot, int group, int8_t* q, float* s) {
    return sq_run(x, x_dt, M, C, x_dt, rot, group, 0, q, s);
}

typedef struct {
    const void* x; int x_dt; int64_t C; int norm; const float* w; const float* b; float eps; const int32_t* rows;
    const void* scale; const void* shift; const void* gate; int tab_dt; int act; const void* res; int res_dt; void* out;
    int out_dt;
} nmag_ctx;
static void nmag_rows(void* p, int64_t r0, int64_t r1) {
    const nmag_ctx* c = (const nmag_ctx*) p;
    const int64_t C = c->C;
    const int V = vec_of(c->x_dt);
    float* row = (float*) malloc((size_t) C * sizeof(float));
    for (int64_t r = r0; r < r1; ++r) {
        for (int64_t i = 0; i < C; ++i) row[i] = h3o_load(c->x, c->x_dt, r * C + i);
        float mean = 0.0f, inv;
        if (c->norm == H3O_NORM_LAYER) ln_stats(row, C, V, c->eps, &mean, &inv);
        else inv = inv_root(h3o_canon_sum(row, C, V, h3o_row_lanes(C, V), H3O_SUMSQ, 0.0f), C, c->eps);
        const int64_t tr = c->rows ? c->rows[r] : 0;
        for (int64_t i = 0; i < C; ++i) {
            float v = c->norm == H3O_NORM_LAYER ? (row[i] - mean) * inv : row[i] * inv;
            if (c->w) v = v * c->w[i];
            if (c->b) v = v + c->b[i];
            if (c->scale && c->shift) {
                const float sc = h3o_load(c->scale, c->tab_dt, tr * C + i), sh = h3o_load(c->shift, c->tab_dt, tr * C + i);
                v = v * (1.0f + sc) + sh;
            }
            v = h3o_act(v, c->act);
            if (c->gate) v = v * h3o_load(c->gate, c->tab_dt, tr * C + i);
            if (c->res) v = h3o_load(c->res, c->res_dt, r * C + i) + v;
            h3o_store(c->out, c->out_dt, r * C + i, v);
        }
    }
    free(row);
}
int h3o_norm_mod_act_gate(const void* x, int x_dt, int64_t M, int64_t C, int norm, const float* weight,
                          const float* bias, float eps, const int32_t* rows, const void* scale, const void* shift,
                          const void* gate, int tab_dt, int act, const void* res, int res_dt, void* out, int out_dt) {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(tab_dt) || !dt_ok(res_dt) || !dt_ok(out_dt)) return fail("norm_mod_act_gate: unknown element type");
    nmag_ctx c = {x, x_dt, C, norm, weight, bias, eps, rows, scale, shift, gate, tab_dt, act, res, res_dt, out, out_dt};
    parallel_rows(M, nmag_rows, &c);
    return 0;
}

/* ---- reference::compare: engine/h3-core/src/reference.rs:84-95 ---- */
/* ---- attention: kernels/h3sycl.cpp:1676-1767 (sage), 1496-1550 (16-bit) ---- */
void h3o_sage_quantize(const void* src, int dt, int64_t S, int64_t H, int64_t D, int64_t stride, const float* mean,
                       int8_t* codes, float* scales) {
    const int64_t nb = (S + 63) / 64;
    for (int64_t h = 0; h < H; ++h)
        for (int64_t b = 0; b < nb; ++b) {
            const int64_t r0 = b * 64, rows = S - r0 < 64 ? S - r0 : 64;
            float m = 0.0f;                                                      /* h3sycl.cpp:1738-1742 */
            for (int64_t r = r0; r < r0 + rows; ++r)
                for (int64_t d = 0; d < D; ++d) {
                    const float x = fabsf(h3o_load(src, dt, r * stride + h * D + d) - (mean ? mean[h * D + d] : 0.0f));
                    m = fmaxf(m, x);
                }
            const float inv = m > 0.0f ? 127.0f / m : 0.0f;                      /* h3sycl.cpp:1744-1745 */
            scales[h * nb + b] = m / 127.0f;
            for (int64_t r = r0; r < r0 + rows; ++r)
                for (int64_t d = 0; d < D; ++d) {
                    const float x = (h3o_load(src, dt, r * stride + h * D + d) - (mean ? mean[h * D + d] : 0.0f)) * inv;
                    float c = roundf(x);                                         /* sycl::round: half away from zero */
                    c = c < -127.0f ? -127.0f : c > 127.0f ? 127.0f : c;
                    codes[(h * S + r) * D + d] = (int8_t) c;
                }
        }
}

typedef struct {
    int64_t S, H, D;
    int sage;
    const int8_t* iq; const int8_t* ik; const float* qs; const float* ks;   /* sage */
    const float* hq; const float* hk;                                       /* 16-bit: half values as float */
    const float* hv;                                                        /* [H, S, D] half values as float */
    float scale;
    void* out; int out_dt;
} attn_ctx;
static void attn_rows(void* p, int64_t r0, int64_t r1) {
    const attn_ctx* c = (const attn_ctx*) p;
    const int64_t S = c->S, H = c->H, D = c->D, nb = (S + 63) / 64;
    double* sc = (double*) malloc((size_t) S * sizeof(double));
    double* acc = (double*) malloc((size_t) D * sizeof(double));
    for (int64_t t = r0; t < r1; ++t)                 /* a row of the [S * H] (token, head) pairs */
    {
        const int64_t i = t / H, h = t % H;
        double mx = -1e300;
        for (int64_t j = 0; j < S; ++j) {
            double v;
            if (c->sage) {
                int64_t a = 0;
                const int8_t* qi = c->iq + (h * S + i) * D;
                const int8_t* kj = c->ik + (h * S + j) * D;
                for (int64_t d = 0; d < D; ++d) a += (int64_t) qi[d] * kj[d];
                v = (double) a * c->qs[h * nb + i / 64] * c->ks[h * nb + j / 64] * c->scale;
            } else {
                double a = 0.0;
                const float* qi = c->hq + (h * S + i) * D;
                const float* kj = c->hk + (h * S + j) * D;
                for (int64_t d = 0; d < D; ++d) a += (double) qi[d] * kj[d];
                v = a * c->scale;
            }
            sc[j] = v;
            if (v > mx) mx = v;
        }
        double l = 0.0;
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
        for (int64_t j = 0; j < S; ++j) {
            const double w = exp(sc[j] - mx);
            l += w;
            const float* vj = c->hv + (h * S + j) * D;
            for (int64_t d = 0; d < D; ++d) acc[d] += w * vj[d];
        }
        for (int64_t d = 0; d < D; ++d) {
            const float ao = h3o_f16_to_f32(h3o_f32_to_f16((float) (acc[d] / l)));   /* the half result buffer */
            h3o_store(c->out, c->out_dt, (i * H + h) * D + d, ao);
        }
    }
    free(sc);
    free(acc);
}
int h3o_attention(const void* q, const void* k, const void* v, int dt, int64_t S, int64_t H, int64_t D, int64_t stride,
                  void* out, int out_dt, int sage, int8_t* iq, int8_t* ik, float* qs, float* ks, float* kmean) {
    if (S <= 0 || H <= 0 || D <= 0) return 0;
    if (!dt_ok(dt) || !dt_ok(out_dt)) return fail("attention: unknown element type");
    if (stride < H * D) return fail("attention: the row stride is shorter than a row");
    const int64_t n = S * H * D, nb = (S + 63) / 64;
    float* hv = (float*) malloc((size_t) n * sizeof(float));
    for (int64_t h = 0; h < H; ++h)
        for (int64_t t = 0; t < S; ++t)
            for (int64_t d = 0; d < D; ++d)
                hv[(h * S + t) * D + d] = h3o_f16_to_f32(h3o_f32_to_f16(h3o_load(v, dt, t * stride + h * D + d)));
    attn_ctx c = {S, H, D, sage, NULL, NULL, NULL, NULL, NULL, NULL, hv, 1.0f / sqrtf((float) D), out, out_dt};
    int8_t *bq = NULL, *bk = NULL;
    float *bqs = NULL, *bks = NULL, *bm = NULL, *fq = NULL, *fk = NULL;
    if (sage) {
        bq = iq ? iq : (int8_t*) malloc((size_t) n);
        bk = ik ? ik : (int8_t*) malloc((size_t) n);
        bqs = qs ? qs : (float*) malloc((size_t) (H * nb) * sizeof(float));
        bks = ks ? ks : (float*) malloc((size_t) (H * nb) * sizeof(float));
        bm = kmean ? kmean : (float*) malloc((size_t) (H * D) * sizeof(float));
        for (int64_t hd = 0; hd < H * D; ++hd) {                                  /* h3sycl.cpp:1729-1733 */
            float sum = 0.0f;
            for (int64_t t = 0; t < S; ++t) sum += h3o_load(k, dt, t * stride + hd);
            bm[hd] = sum / (float) S;
        }
        h3o_sage_quantize(q, dt, S, H, D, stride, NULL, bq, bqs);
        h3o_sage_quantize(k, dt, S, H, D, stride, bm, bk, bks);
        c.iq = bq; c.ik = bk; c.qs = bqs; c.ks = bks;
    } else {
        fq = (float*) malloc((size_t) n * sizeof(float));
        fk = (float*) malloc((size_t) n * sizeof(float));
        for (int64_t h = 0; h < H; ++h)
            for (int64_t t = 0; t < S; ++t)
                for (int64_t d = 0; d < D; ++d) {
                    fq[(h * S + t) * D + d] = h3o_f16_to_f32(h3o_f32_to_f16(h3o_load(q, dt, t * stride + h * D + d)));
                    fk[(h * S + t) * D + d] = h3o_f16_to_f32(h3o_f32_to_f16(h3o_load(k, dt, t * stride + h * D + d)));
                }
        c.hq = fq; c.hk = fk;
    }
    parallel_rows(S * H, attn_rows, &c);
    free(hv);
    free(fq);
    free(fk);
    if (sage) {
        if (!iq) free(bq);
        if (!ik) free(bk);
        if (!qs) free(bqs);
        if (!ks) free(bks);
        if (!kmean) free(bm);
    }
    return 0;
}

/* ---- causal attention: kernels/h3sycl.cpp:873-898 ---- */
typedef struct { const void *q, *k, *v; int dt; int64_t L, Hq, Hkv, D, qs, kvs; void* out; } causal_ctx;
static void causal_rows(void* p, int64_t r0, int64_t r1) {
    const causal_ctx* c = (const causal_ctx*) p;
    const int64_t D = c->D;
    double* sc = (double*) malloc((size_t) c->L * sizeof(double));
    double* acc = (double*) malloc((size_t) D * sizeof(double));
    const double scale = 1.0f / sqrtf((float) D);
    for (int64_t t = r0; t < r1; ++t) {
        const int64_t i = t / c->Hq, h = t % c->Hq, g = h / (c->Hq / c->Hkv);
        double mx = -1e300;
        for (int64_t j = 0; j <= i; ++j) {
            double a = 0.0;
            for (int64_t d = 0; d < D; ++d)
                a += (double) h3o_load(c->q, c->dt, i * c->qs + h * D + d) * h3o_load(c->k, c->dt, j * c->kvs + g * D + d);
            sc[j] = a * scale;
            if (sc[j] > mx) mx = sc[j];
        }
        double l = 0.0;
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
        for (int64_t j = 0; j <= i; ++j) {
            const double w = exp(sc[j] - mx);
            l += w;
            for (int64_t d = 0; d < D; ++d) acc[d] += w * h3o_load(c->v, c->dt, j * c->kvs + g * D + d);
        }
        for (int64_t d = 0; d < D; ++d) h3o_store(c->out, c->dt, (i * c->Hq + h) * D + d, (float) (acc[d] / l));
    }
    free(sc);
    free(acc);
}
int h3o_attention_causal(const void* q, const void* k, const void* v, int dt, int64_t L, int64_t Hq, int64_t Hkv, int64_t D,
                         int64_t qs, int64_t kvs, void* out) {
    if (L <= 0) return 0;
    if (Hq % Hkv != 0) return fail("attention_causal: Hq a multiple of Hkv");
    causal_ctx c = {q, k, v, dt, L, Hq, Hkv, D, qs, kvs, out};
    parallel_rows(L * Hq, causal_rows, &c);
    return 0;
}

/* ---- plain linear layers: kernels/h3sycl.cpp:656-739 ---- */
typedef struct { const void* x; int dt; int64_t K; const void* w; int64_t N; const float* bias; void* out; int out_dt; int acc; } lin_ctx;
static void lin_rows(void* p, int64_t r0, int64_t r1) {
    const lin_ctx* c = (const lin_ctx*) p;
    for (int64_t r = r0; r < r1; ++r)
        for (int64_t n = 0; n < c->N; ++n) {
            double a = 0.0;
            for (int64_t k = 0; k < c->K; ++k) a += (double) h3o_load(c->x, c->dt, r * c->K + k) * h3o_load(c->w, c->dt, n * c->K + k);
            float v = (float) a;
            if (c->bias) v = v + c->bias[n];
            if (c->acc) v = v + h3o_load(c->out, c->out_dt, r * c->N + n);
            h3o_store(c->out, c->out_dt, r * c->N + n, v);
        }
}
void h3o_linear(const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N, const float* bias, void* out,
                int out_dt, int acc) {
    lin_ctx c = {x, dt, K, w, N, bias, out, out_dt, acc};
    parallel_rows(M, lin_rows, &c);
}
void h3o_scale_rows(void* x, int dt, int64_t M, int64_t C, const float* s) {
    for (int64_t r = 0; r < M; ++r)
        for (int64_t i = 0; i < C; ++i) h3o_store(x, dt, r * C + i, h3o_load(x, dt, r * C + i) * s[r]);
}

/* ---- a step's tables: engine/h3-core/src/dit.rs:155-174 and 188-203 ---- */
void h3o_adaln_tables(const float* w, const float* b, const float* t_emb, int64_t R, int64_t t_dim, int64_t m, int64_t C,
                      float* out) {
    for (int64_t r = 0; r < R; ++r)
        for (int64_t mi = 0; mi < m; ++mi)
            for (int64_t ci = 0; ci < 6; ++ci)
                for (int64_t i = 0; i < C; ++i) {
                    const int64_t o = mi * 6 * C + ci * C + i;
                    float sum = -0.0f;                                   /* dit.rs:168-169: iter().zip().map().sum() */
                    for (int64_t k = 0; k < t_dim; ++k) sum = sum + w[o * t_dim + k] * t_emb[r * t_dim + k];
                    out[ci * R * m * C + (r * m + mi) * C + i] = b[o] + sum;
                }
}
void h3o_rotations(const double* positions, int64_t S, const float* inv_freq, int64_t n, float* cs) {
    float* p = cs;
    for (int64_t s = 0; s < S; ++s)
        for (int a = 0; a < 3; ++a)
            for (int64_t f = 0; f < n; ++f) {
                const float ang = (float) positions[s * 3 + a] * inv_freq[f];   /* dit.rs:196 */
                *p++ = cosf(ang);
                *p++ = sinf(ang);
            }
}

/* ---- token layout: engine/h3-core/src/layout.rs:88-176 (Layout::new), appended row by row in its order ---- */
typedef struct { double* pos; int32_t* kind; int64_t n, cap; } lay_out;
static void lay_put(lay_out* o, double t, double h, double w, int32_t kind) {
    if (o->n < o->cap) {
        if (o->pos) { o->pos[3 * o->n] = t; o->pos[3 * o->n + 1] = h; o->pos[3 * o->n + 2] = w; }
        if (o->kind) o->kind[o->n] = kind;
    }
    ++o->n;
}
static double lay_axis(int64_t dim, double sqrt_area, int64_t i) {                             /* layout.rs:89-93 */
    const double ratio = (double) dim / sqrt_area;
    const int64_t n = dim / 2;
    return ((double) i * (ratio / (double) n) + (1.0 - ratio) / 2.0) * 32.0;
}
static void lay_video(lay_out* o, int64_t vt, double origin, int64_t H, int64_t W, double sa, int32_t kind) {
    static const double per[5] = {1.0, 4.0, 4.0, 4.0, 4.0};                                    /* layout.rs:15-16 */
    double t = origin;
    for (int64_t k = 0; k < vt; ++k) {                                                          /* layout.rs:96-105 */
        for (int64_t a = 0; a < H / 2; ++a)
            for (int64_t b = 0; b < W / 2; ++b) lay_put(o, t, lay_axis(H, sa, a), lay_axis(W, sa, b), kind);
        t += 5.0 / 3.0 * per[k % 5];
    }
}
static void lay_audio(lay_out* o, int64_t at, double origin, int64_t W, double sa, int32_t kind) {   /* layout.rs:134-140 */
    const double ends[2] = {lay_axis(W, sa, 0), lay_axis(W, sa, W / 2 - 1)};
    for (int c = 0; c < 2; ++c)
        for (int64_t i = 0; i < at; ++i) lay_put(o, origin + (double) i, 0.0, ends[c], kind);
}
int64_t h3o_layout(int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
                   const double* kf_index, const int64_t* kf_video, const int64_t* kf_audio, int64_t n_kf,
                   const int64_t* ref_audio, int64_t n_refs, double* positions, int32_t* kinds, int64_t cap) {
    if (latent_h <= 0 || latent_w <= 0 || latent_h % 2 || latent_w % 2) return fail("layout: even latent height and width");
    const double sa = sqrt((double) (latent_h * latent_w));
    lay_out o = {positions, kinds, 0, cap};
    for (int64_t i = 0; i < text_len; ++i) lay_put(&o, (double) i, 0.0, 0.0, H3O_TOK_TEXT);     /* layout.rs:142-145 */
    double spans = 0.0;
    for (int64_t r = 0; r < n_refs; ++r) spans += (double) ref_audio[r];
    const double cursor = (double) text_len + spans;                                            /* layout.rs:147 */
    for (int64_t k = 0; k < n_kf; ++k) {                                                        /* layout.rs:148-158 */
        const double at = cursor + 5.0 / 3.0 * kf_index[k];
        if (kf_video[k] >= 0) lay_video(&o, kf_video[k], at, latent_h, latent_w, sa, H3O_TOK_COND);
        if (kf_audio[k] >= 0) lay_audio(&o, kf_audio[k], at, latent_w, sa, H3O_TOK_COND_AUDIO);
    }
    double rc = (double) text_len;                                                              /* layout.rs:159-170 */
    for (int64_t r = 0; r < n_refs; ++r) {
        if (ref_audio[r] > 0) lay_audio(&o, ref_audio[r], rc, latent_w, sa, H3O_TOK_REF_AUDIO);
        rc += (double) ref_audio[r];
    }
    lay_audio(&o, audio_t, cursor, latent_w, sa, H3O_TOK_AUDIO);                               /* layout.rs:171-174 */
    lay_video(&o, latent_t, cursor, latent_h, latent_w, sa, H3O_TOK_VIDEO);
    return o.n;
}

void h3o_compare(const float* a, const float* b, int64_t n, double* rel, double* cos) {
    double d2 = 0, a2 = 0, b2 = 0, ab = 0;
    for (int64_t i = 0; i < n; ++i) {
        const double x = a[i], y = b[i];
        d2 += (x - y) * (x - y);
        a2 += x * x;
        b2 += y * y;
        ab += x * y;
    }
    *rel = sqrt(d2 / (b2 > 1e-300 ? b2 : 1e-300));
    const double den = sqrt(a2) * sqrt(b2);
    *cos = ab / (den > 1e-300 ? den : 1e-300);
}
