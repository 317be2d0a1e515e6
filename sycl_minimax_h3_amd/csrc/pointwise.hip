// pointwise.hip - h3s_swiglu (kernels/h3sycl.cpp:1378-1419) and h3s_gate_add (kernels/h3sycl.cpp:1421-1431): 16-byte
// chunks of a row, up to eight a thread, a block a row (or a run of 2048 chunks of one).
#include <algorithm>

#include "rowcore.h"

namespace h3 {

template <int V> __device__ __forceinline__ void load_rt(const void* p, int dt, int64_t i, float* f) {
    if (dt == H3S_F32) load_f32x((const float*) p + i, f, V);
    else if (dt == H3S_BF16) load_tab<H3S_BF16>(p, i, f, V);
    else load_tab<H3S_F16>(p, i, f, V);
}
// (nontemporal stores: the outputs are streamed, never read back here)
template <int V> __device__ __forceinline__ void store_rt2(void* out, int out_dt, int64_t i, const float* f) {
    if (out_dt == H3S_F32) {
#pragma unroll
        for (int k = 0; k < V; k += 4)
            st_nt((float*) out + i + k, make_uint4(__float_as_uint(f[k]), __float_as_uint(f[k + 1]), __float_as_uint(f[k + 2]),
                                                   __float_as_uint(f[k + 3])));
    } else {
        uint32_t w[V / 2];
#pragma unroll
        for (int k = 0; k < V; k += 2) w[k / 2] = out_dt == H3S_BF16 ? pack_bf16(f[k], f[k + 1]) : pack_f16(f[k], f[k + 1]);
        uint16_t* o = (uint16_t*) out + i;
        if constexpr (V == 8) st_nt(o, make_uint4(w[0], w[1], w[2], w[3]));
        else st_nt(o, make_uint2(w[0], w[1]));
    }
}

// The grid is a 1-D run of (row, column block) pairs: block b takes row b / cb of the output and its 16-byte chunks
// (b % cb) 256 K + t + 256 k (k < K) for thread t (cb blocks a row), their loads in flight together; K is the row's
// chunks / 256 rounded up, at most 8 (4 for gate_add, whose three inputs hold more registers a chunk), so a row is
// one block where it can be (5376 features: 672 chunks, K = 3; 14336: 1792, K = 7). The row of a block is one scalar
// division, no per-chunk 64-bit division.
constexpr int kPwThreads = 256;

// out[r, i] = silu(x[r, i]) * x[r, C + i]
template <int XDT, int kPwChunks>
__global__ __launch_bounds__(kPwThreads) void swiglu_kernel(const void* __restrict__ x, int64_t M, int64_t C, void* __restrict__ out,
                                                            int out_dt, int cb) {
    constexpr int V = Vec<XDT>::V;
    const int64_t r = blockIdx.x / (unsigned) cb;
    const int64_t cpr = C / V, c0 = (int64_t) (blockIdx.x - r * cb) * (kPwThreads * kPwChunks) + threadIdx.x;
    const uint4* xr = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(x) + r * 2 * C * (16 / V));
    uint4 g[kPwChunks], u[kPwChunks];
#pragma unroll
    for (int k = 0; k < kPwChunks; ++k) {
        const int64_t c = c0 + k * kPwThreads;
        if (c < cpr) {
            g[k] = ld_nt(xr + c);
            u[k] = ld_nt(xr + cpr + c);
        }
    }
#pragma unroll
    for (int k = 0; k < kPwChunks; ++k) {
        const int64_t c = c0 + k * kPwThreads;
        if (c >= cpr) continue;
        float gv[V], uv[V], o[V];
        Vec<XDT>::unpack(g[k], gv);
        Vec<XDT>::unpack(u[k], uv);
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = act_silu(gv[e]) * uv[e];
        store_rt2<V>(out, out_dt, r * C + c * V, o);
    }
}

// x[r, i] += other[r, i] * gate[rows[r] * C + i]  (gate NULL: 1)
template <int XDT, int kPwChunks>
__global__ __launch_bounds__(kPwThreads) void gate_add_kernel(void* x, int64_t M, int64_t C, const void* other, int other_dt,
                                                              const int32_t* __restrict__ rows, const float* __restrict__ gate,
                                                              int cb) {
    constexpr int V = Vec<XDT>::V;
    const int64_t r = blockIdx.x / (unsigned) cb;
    const int64_t cpr = C / V, c0 = (int64_t) (blockIdx.x - r * cb) * (kPwThreads * kPwChunks) + threadIdx.x;
    uint4* xr = reinterpret_cast<uint4*>(reinterpret_cast<char*>(x) + r * C * (16 / V));
    const float* grow = gate ? gate + (int64_t) rows[r] * C : nullptr;
    uint4 a[kPwChunks];
    float b[kPwChunks][V], gv[kPwChunks][V];
#pragma unroll
    for (int k = 0; k < kPwChunks; ++k) {
        const int64_t c = c0 + k * kPwThreads;
        if (c < cpr) {
            a[k] = ld_nt(xr + c);
            load_rt<V>(other, other_dt, r * C + c * V, b[k]);
            if (grow) load_f32x(grow + c * V, gv[k], V);
        }
    }
#pragma unroll
    for (int k = 0; k < kPwChunks; ++k) {
        const int64_t c = c0 + k * kPwThreads;
        if (c >= cpr) continue;
        float av[V];
        Vec<XDT>::unpack(a[k], av);
        if (grow) {
#pragma unroll
            for (int e = 0; e < V; ++e) av[e] = av[e] + b[k][e] * gv[k][e];
        } else {
#pragma unroll
            for (int e = 0; e < V; ++e) av[e] = av[e] + b[k][e] * 1.0f;
        }
        st_nt(xr + c, Vec<XDT>::pack(av));
    }
}

// chunks a thread (K, at most maxk) and column blocks a row
static int pw_chunks(int64_t C, int V, int maxk) { return (int) std::min<int64_t>(maxk, (C / V + kPwThreads - 1) / kPwThreads); }
static int pw_blocks_a_row(int64_t C, int V, int K) { return (int) ((C / V + kPwThreads * K - 1) / (kPwThreads * K)); }
static bool pw_grid_ok(int64_t M, int cb) { return M * cb <= 0x7fffffff; }
#define H3_PW_K(KK, LAUNCH)       \
    switch (KK) {                 \
        case 1: LAUNCH(1); break; \
        case 2: LAUNCH(2); break; \
        case 3: LAUNCH(3); break; \
        case 4: LAUNCH(4); break; \
        case 5: LAUNCH(5); break; \
        case 6: LAUNCH(6); break; \
        case 7: LAUNCH(7); break; \
        default: LAUNCH(8); break; \
    }
#define H3_PW_K4(KK, LAUNCH)      \
    switch (KK) {                 \
        case 1: LAUNCH(1); break; \
        case 2: LAUNCH(2); break; \
        case 3: LAUNCH(3); break; \
        default: LAUNCH(4); break; \
    }

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_swiglu(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, void* out, int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(out_dt)) return fail("h3s_swiglu: unknown element type");
    const int V = vec_of(x_dt);
    if (C % V != 0) return fail("h3s_swiglu: C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors)");
    if (!aligned16(x) || !aligned16(out)) return fail("h3s_swiglu: tensors must be 16-byte aligned");
    const int K = pw_chunks(C, V, 8), cb = pw_blocks_a_row(C, V, K);
    if (!pw_grid_ok(M, cb)) return fail("h3s_swiglu: too many rows");
    Ctx* c = ctx_of(ctx, "h3s_swiglu");
    if (!c) return -1;
    const unsigned g = (unsigned) (M * cb);
#define H3_SW(KK)                                                                                                        \
    switch (x_dt) {                                                                                                      \
        case H3S_BF16: swiglu_kernel<H3S_BF16, KK><<<g, kPwThreads, 0, c->stream>>>(x, M, C, out, out_dt, cb); break;   \
        case H3S_F16: swiglu_kernel<H3S_F16, KK><<<g, kPwThreads, 0, c->stream>>>(x, M, C, out, out_dt, cb); break;     \
        default: swiglu_kernel<H3S_F32, KK><<<g, kPwThreads, 0, c->stream>>>(x, M, C, out, out_dt, cb); break;          \
    }
    H3_PW_K(K, H3_SW)
#undef H3_SW
    return launched("h3s_swiglu");
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_gate_add(void* ctx, void* x, int x_dt, int64_t M, int64_t C, const void* other, int other_dt,
                            const int32_t* rows, const float* gate) try {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(other_dt)) return fail("h3s_gate_add: unknown element type");
    if (gate && !rows) return fail("h3s_gate_add: a gate needs the row table");
    const int V = vec_of(x_dt);
    if (C % V != 0) return fail("h3s_gate_add: C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors)");
    if (!aligned16(x) || !aligned16(other) || (gate && !aligned16(gate))) return fail("h3s_gate_add: tensors must be 16-byte aligned");
    const int K = pw_chunks(C, V, 4), cb = pw_blocks_a_row(C, V, K);
    if (!pw_grid_ok(M, cb)) return fail("h3s_gate_add: too many rows");
    Ctx* c = ctx_of(ctx, "h3s_gate_add");
    if (!c) return -1;
    const unsigned g = (unsigned) (M * cb);
#define H3_GA(KK)                                                                                                                 \
    switch (x_dt) {                                                                                                               \
        case H3S_BF16: gate_add_kernel<H3S_BF16, KK><<<g, kPwThreads, 0, c->stream>>>(x, M, C, other, other_dt, rows, gate, cb); break; \
        case H3S_F16: gate_add_kernel<H3S_F16, KK><<<g, kPwThreads, 0, c->stream>>>(x, M, C, other, other_dt, rows, gate, cb); break;   \
        default: gate_add_kernel<H3S_F32, KK><<<g, kPwThreads, 0, c->stream>>>(x, M, C, other, other_dt, rows, gate, cb); break;        \
    }
    H3_PW_K4(K, H3_GA)
#undef H3_GA
    return launched("h3s_gate_add");
} catch (const std::exception& e) { return fail(e.what()); }
