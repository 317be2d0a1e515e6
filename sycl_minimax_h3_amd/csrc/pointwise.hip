// pointwise.hip - h3s_swiglu (kernels/h3sycl.cpp:1378-1419) and h3s_gate_add (kernels/h3sycl.cpp:1421-1431): one
// 16-byte chunk of the row per thread, grid-stride over the whole tensor.
#include "rowcore.h"

namespace h3 {

template <int V> __device__ __forceinline__ void load_rt(const void* p, int dt, int64_t i, float* f) {
    if (dt == H3S_F32) load_f32x((const float*) p + i, f, V);
    else if (dt == H3S_BF16) load_tab<H3S_BF16>(p, i, f, V);
    else load_tab<H3S_F16>(p, i, f, V);
}
template <int V> __device__ __forceinline__ void store_rt2(void* out, int out_dt, int64_t i, const float* f) {
    if (out_dt == H3S_F32) {
#pragma unroll
        for (int k = 0; k < V; k += 4)
            *reinterpret_cast<float4*>((float*) out + i + k) = make_float4(f[k], f[k + 1], f[k + 2], f[k + 3]);
    } else {
        uint32_t w[V / 2];
#pragma unroll
        for (int k = 0; k < V; k += 2) w[k / 2] = out_dt == H3S_BF16 ? pack_bf16(f[k], f[k + 1]) : pack_f16(f[k], f[k + 1]);
        uint16_t* o = (uint16_t*) out + i;
        if constexpr (V == 8) *reinterpret_cast<uint4*>(o) = make_uint4(w[0], w[1], w[2], w[3]);
        else *reinterpret_cast<uint2*>(o) = make_uint2(w[0], w[1]);
    }
}

// out[r, i] = silu(x[r, i]) * x[r, C + i]
template <int XDT>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ x, int64_t M, int64_t C, void* __restrict__ out,
                                                     int out_dt) {
    constexpr int V = Vec<XDT>::V;
    const int64_t cpr = C / V, n = M * cpr;
    for (int64_t k = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t) gridDim.x * blockDim.x) {
        const int64_t r = k / cpr, i = (k - r * cpr) * V;
        const uint4* xr = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(x) + r * 2 * C * (16 / V));
        float g[V], u[V], o[V];
        Vec<XDT>::unpack(ld_nt(xr + i / V), g);
        Vec<XDT>::unpack(ld_nt(xr + (C + i) / V), u);
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = act_silu(g[e]) * u[e];
        store_rt2<V>(out, out_dt, r * C + i, o);
    }
}

// x[r, i] += other[r, i] * gate[rows[r] * C + i]  (gate NULL: 1)
template <int XDT>
__global__ __launch_bounds__(256) void gate_add_kernel(void* x, int64_t M, int64_t C, const void* other, int other_dt,
                                                       const int32_t* __restrict__ rows, const float* __restrict__ gate) {
    constexpr int V = Vec<XDT>::V;
    const int64_t cpr = C / V, n = M * cpr;
    for (int64_t k = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t) gridDim.x * blockDim.x) {
        const int64_t r = k / cpr, i = (k - r * cpr) * V, p = r * C + i;
        uint4* xp = reinterpret_cast<uint4*>(reinterpret_cast<char*>(x) + p * (16 / V));
        float a[V], b[V];
        Vec<XDT>::unpack(ld_nt(xp), a);
        load_rt<V>(other, other_dt, p, b);
        if (gate) {
            float g[V];
            load_f32x(gate + (int64_t) rows[r] * C + i, g, V);
#pragma unroll
            for (int e = 0; e < V; ++e) a[e] = a[e] + b[e] * g[e];
        } else {
#pragma unroll
            for (int e = 0; e < V; ++e) a[e] = a[e] + b[e] * 1.0f;
        }
        *xp = Vec<XDT>::pack(a);
    }
}

static unsigned grid_for(int64_t chunks, const Ctx& c) {
    (void) c;
    const int64_t blocks = (chunks + 255) / 256;
    return (unsigned) (blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_swiglu(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, void* out, int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(x_dt) || !dt_ok(out_dt)) return fail("h3s_swiglu: unknown element type");
    const int V = vec_of(x_dt);
    if (C % V != 0) return fail("h3s_swiglu: C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors)");
    if (!aligned16(x) || !aligned16(out)) return fail("h3s_swiglu: tensors must be 16-byte aligned");
    Ctx* c = ctx_of(ctx, "h3s_swiglu");
    if (!c) return -1;
    const unsigned g = grid_for(M * (C / V), *c);
    switch (x_dt) {
        case H3S_BF16: swiglu_kernel<H3S_BF16><<<g, 256, 0, c->stream>>>(x, M, C, out, out_dt); break;
        case H3S_F16: swiglu_kernel<H3S_F16><<<g, 256, 0, c->stream>>>(x, M, C, out, out_dt); break;
        default: swiglu_kernel<H3S_F32><<<g, 256, 0, c->stream>>>(x, M, C, out, out_dt); break;
    }
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
    Ctx* c = ctx_of(ctx, "h3s_gate_add");
    if (!c) return -1;
    const unsigned g = grid_for(M * (C / V), *c);
    switch (x_dt) {
        case H3S_BF16: gate_add_kernel<H3S_BF16><<<g, 256, 0, c->stream>>>(x, M, C, other, other_dt, rows, gate); break;
        case H3S_F16: gate_add_kernel<H3S_F16><<<g, 256, 0, c->stream>>>(x, M, C, other, other_dt, rows, gate); break;
        default: gate_add_kernel<H3S_F32><<<g, 256, 0, c->stream>>>(x, M, C, other, other_dt, rows, gate); break;
    }
    return launched("h3s_gate_add");
} catch (const std::exception& e) { return fail(e.what()); }
