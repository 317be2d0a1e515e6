// rownorm.hip - the per-token row kernels: h3s_rms_norm_mod, h3s_layer_norm (kernels/h3sycl.cpp:766-810,
// 1248-1274), and the fused chains h3s_norm_quant (rms_norm_mod -> bf16 h -> int8_linear's quantizer,
// engine/h3-core/src/dit.rs:340-342 with kernels/h3sycl.cpp:404-474) and h3s_norm_mod_act_gate.
//
// One 64-wide wavefront per token row, four rows per 256-thread workgroup. The row is read once through 16-byte
// loads: lane l holds the 16-byte chunks l, l + 64, l + 128, ... (CPL of them, in registers), so each load
// instruction of the wave covers 1 KiB of consecutive bytes. Row statistics are a per-lane sum in chunk order then
// an xor butterfly across the 64 lanes: the canonical order the CPU oracle follows. Every output is written once.
#include "common.h"

namespace h3 {

template <int XDT, int CPL> struct RowRegs {
    static constexpr int V = Vec<XDT>::V;
    float v[CPL][V];
    int64_t nch;   // 16-byte chunks in the row

    __device__ __forceinline__ void load(const void* x, int64_t row, int64_t C, int lane) {
        nch = C / V;
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(x) + row * C * (16 / V));
        uint4 raw[CPL];
        // every lane loads (a chunk past the row's end reads the last one again and is never used): no branch
        // between the loads, so all of them are in flight together
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + (int64_t) kWave * j;
            raw[j] = p[c < nch ? c : nch - 1];
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) Vec<XDT>::unpack(raw[j], v[j]);
    }
    __device__ __forceinline__ bool valid(int lane, int j) const { return lane + (int64_t) kWave * j < nch; }
    // canonical sums: this lane's chunks in order, then the butterfly
    __device__ __forceinline__ float sum(int lane) const {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (valid(lane, j))
#pragma unroll
                for (int e = 0; e < V; ++e) s = s + v[j][e];
        return wave_sum<kWave>(s);
    }
    __device__ __forceinline__ float sumsq(int lane) const {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (valid(lane, j))
#pragma unroll
                for (int e = 0; e < V; ++e) s = __builtin_fmaf(v[j][e], v[j][e], s);
        return wave_sum<kWave>(s);
    }
    __device__ __forceinline__ float sumsq_diff(int lane, float mean) const {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (valid(lane, j))
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float d = v[j][e] - mean;
                    s = __builtin_fmaf(d, d, s);
                }
        return wave_sum<kWave>(s);
    }
};

// V values of a table row in tab_dt (F32 or BF16)
template <int V> __device__ __forceinline__ void load_tab_rt(const void* t, int tab_dt, int64_t i, float* f) {
    if (tab_dt == H3S_F32) load_tab<H3S_F32>(t, i, f, V);
    else if (tab_dt == H3S_BF16) load_tab<H3S_BF16>(t, i, f, V);
    else load_tab<H3S_F16>(t, i, f, V);
}

// V values stored as the chunk starting at element i of out, in out_dt
template <int V> __device__ __forceinline__ void store_rt(void* out, int out_dt, int64_t i, const float* f) {
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

__device__ __forceinline__ float round_rt(float v, int dt) {
    if (dt == H3S_BF16) return round_bf16(v);
    if (dt == H3S_F16) return round_f16(v);
    return v;
}

// ---- h3s_rms_norm_mod: inv = 1/sqrt(sum x^2 / C + eps); out = x * inv * w [* (1 + scale[t]) + shift[t]] ----
template <int XDT, int CPL>
__global__ __launch_bounds__(256) void rms_norm_mod_kernel(const void* __restrict__ x, int64_t M, int64_t C,
                                                           const float* __restrict__ w, float eps,
                                                           const int32_t* __restrict__ rows, const float* __restrict__ scale,
                                                           const float* __restrict__ shift, void* out, int out_dt) {
    constexpr int V = Vec<XDT>::V;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    RowRegs<XDT, CPL> R;
    R.load(x, row, C, lane);
    const float inv = inv_root(R.sumsq(lane), (float) C, eps);
    const int64_t tr = rows ? (int64_t) rows[row] * C : 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if (!R.valid(lane, j)) continue;
        const int64_t i = (lane + (int64_t) kWave * j) * V;
        float wv[V], o[V];
        load_f32x(w + i, wv, V);
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = R.v[j][e] * inv * wv[e];
        if (rows) {
            float sc[V], sh[V];
            load_f32x(scale + tr + i, sc, V);
            load_f32x(shift + tr + i, sh, V);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] * (1.0f + sc[e]) + sh[e];
        }
        store_rt<V>(out, out_dt, row * C + i, o);
    }
}

// ---- h3s_layer_norm: mean, then the centred sum of squares; (x - mean) * inv [* w] [+ b] ----
template <int XDT, int CPL>
__global__ __launch_bounds__(256) void layer_norm_kernel(const void* __restrict__ x, int64_t M, int64_t C,
                                                         const float* __restrict__ w, const float* __restrict__ b, float eps,
                                                         void* out, int out_dt) {
    constexpr int V = Vec<XDT>::V;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    RowRegs<XDT, CPL> R;
    R.load(x, row, C, lane);
    const float mean = R.sum(lane) / (float) C;
    const float inv = inv_root(R.sumsq_diff(lane, mean), (float) C, eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if (!R.valid(lane, j)) continue;
        const int64_t i = (lane + (int64_t) kWave * j) * V;
        float o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = (R.v[j][e] - mean) * inv;
        if (w) {
            float wv[V];
            load_f32x(w + i, wv, V);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] * wv[e];
        }
        if (b) {
            float bv[V];
            load_f32x(b + i, bv, V);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] + bv[e];
        }
        store_rt<V>(out, out_dt, row * C + i, o);
    }
}

// ---- h3s_norm_mod_act_gate: out = res + gate * act(norm(x) [* w] [+ b] [* (1 + scale) + shift]) ----
template <int XDT, int CPL, int ACT, int NORM>
__global__ __launch_bounds__(256) void norm_mod_act_gate_kernel(
    const void* __restrict__ x, int64_t M, int64_t C, const float* __restrict__ w, const float* __restrict__ b, float eps,
    const int32_t* __restrict__ rows, const void* __restrict__ scale, const void* __restrict__ shift,
    const void* __restrict__ gate, int tab_dt, const void* __restrict__ res, int res_dt, void* out, int out_dt) {
    constexpr int V = Vec<XDT>::V;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    RowRegs<XDT, CPL> R;
    R.load(x, row, C, lane);
    // the residual row, issued beside x's loads
    uint4 rraw[CPL];
    const bool res16 = res && res_dt != H3S_F32;
    if (res16) {
        const uint4* rp = reinterpret_cast<const uint4*>((const uint16_t*) res + row * C);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + (int64_t) kWave * j;
            if constexpr (V == 8) rraw[j] = rp[c < R.nch ? c : R.nch - 1];
        }
    }
    float mean = 0.0f, inv;
    if constexpr (NORM == H3S_NORM_LAYER) {
        mean = R.sum(lane) / (float) C;
        inv = inv_root(R.sumsq_diff(lane, mean), (float) C, eps);
    } else {
        inv = inv_root(R.sumsq(lane), (float) C, eps);
    }
    const int64_t tr = rows ? (int64_t) rows[row] * C : 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if (!R.valid(lane, j)) continue;
        const int64_t i = (lane + (int64_t) kWave * j) * V;
        float o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = NORM == H3S_NORM_LAYER ? (R.v[j][e] - mean) * inv : R.v[j][e] * inv;
        if (w) {
            float wv[V];
            load_f32x(w + i, wv, V);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] * wv[e];
        }
        if (b) {
            float bv[V];
            load_f32x(b + i, bv, V);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] + bv[e];
        }
        if (scale && shift) {
            float sc[V], sh[V];
            load_tab_rt<V>(scale, tab_dt, tr + i, sc);
            load_tab_rt<V>(shift, tab_dt, tr + i, sh);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] * (1.0f + sc[e]) + sh[e];
        }
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = act<ACT>(o[e]);
        if (gate) {
            float g[V];
            load_tab_rt<V>(gate, tab_dt, tr + i, g);
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] * g[e];
        }
        if (res) {
            float rv[V];
            if constexpr (V == 8) {
                if (res16) {
                    if (res_dt == H3S_BF16) Vec<H3S_BF16>::unpack(rraw[j], rv);
                    else Vec<H3S_F16>::unpack(rraw[j], rv);
                } else load_f32x((const float*) res + row * C + i, rv, V);
            } else {
                load_tab_rt<V>(res, res_dt, row * C + i, rv);
            }
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = rv[e] + o[e];
        }
        store_rt<V>(out, out_dt, row * C + i, o);
    }
}

// ---- host: shapes, preconditions, instantiation ----
static const char* cpl_error = "rows longer than 16 x 64 16-byte vectors (8192 16-bit or 4096 float32 features) are not supported";

static int cpl_for(int64_t C, int V) {
    const int64_t per_lane = (C / V + kWave - 1) / kWave;
    for (int c : {1, 2, 4, 8, 16})
        if (per_lane <= c) return c;
    return 0;
}
static unsigned grid_rows(int64_t M) { return (unsigned) ((M + 3) / 4); }

#define H3_CPL_SWITCH(cpl, XDT, LAUNCH) \
    switch (cpl) {                        \
        case 1: LAUNCH(XDT, 1); break;    \
        case 2: LAUNCH(XDT, 2); break;    \
        case 4: LAUNCH(XDT, 4); break;    \
        case 8: LAUNCH(XDT, 8); break;    \
        default: LAUNCH(XDT, 16); break;  \
    }
#define H3_DT_SWITCH(dt, cpl, LAUNCH)                                  \
    switch (dt) {                                                      \
        case H3S_BF16: H3_CPL_SWITCH(cpl, H3S_BF16, LAUNCH); break;    \
        case H3S_F16: H3_CPL_SWITCH(cpl, H3S_F16, LAUNCH); break;      \
        default: H3_CPL_SWITCH(cpl, H3S_F32, LAUNCH); break;           \
    }

// the checks every row kernel shares: element types, whole 16-byte vectors per row, alignment, row length
static int row_checks(const char* fn, int x_dt, int out_dt, int64_t C, std::initializer_list<const void*> ptrs, int* cpl) {
    if (!dt_ok(x_dt) || !dt_ok(out_dt)) return fail(std::string(fn) + ": unknown element type");
    const int V = vec_of(x_dt);
    if (C % V != 0)
        return fail(std::string(fn) + ": C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors per row)");
    for (const void* p : ptrs)
        if (p && !aligned16(p)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    *cpl = cpl_for(C, V);
    if (!*cpl) return fail(std::string(fn) + ": " + cpl_error);
    return 0;
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_rms_norm_mod(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps,
                                const int32_t* rows, const float* scale, const float* shift, void* out, int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    int cpl;
    if (row_checks("h3s_rms_norm_mod", x_dt, out_dt, C, {x, weight, scale, shift, out}, &cpl)) return -1;
    if (!weight) return fail("h3s_rms_norm_mod: the weight is required");
    Ctx* c = ctx_of(ctx, "h3s_rms_norm_mod");
    if (!c) return -1;
    const bool mod = rows && scale && shift;
#define L(XDT, CPL)                                                                                                \
    rms_norm_mod_kernel<XDT, CPL><<<grid_rows(M), 256, 0, c->stream>>>(x, M, C, weight, eps, mod ? rows : nullptr, \
                                                                         scale, shift, out, out_dt)
    H3_DT_SWITCH(x_dt, cpl, L)
#undef L
    return launched("h3s_rms_norm_mod");
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_layer_norm(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, const float* bias,
                              float eps, void* out, int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    int cpl;
    if (row_checks("h3s_layer_norm", x_dt, out_dt, C, {x, weight, bias, out}, &cpl)) return -1;
    Ctx* c = ctx_of(ctx, "h3s_layer_norm");
    if (!c) return -1;
#define L(XDT, CPL) layer_norm_kernel<XDT, CPL><<<grid_rows(M), 256, 0, c->stream>>>(x, M, C, weight, bias, eps, out, out_dt)
    H3_DT_SWITCH(x_dt, cpl, L)
#undef L
    return launched("h3s_layer_norm");
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_norm_mod_act_gate(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, int norm, const float* weight,
                                     const float* bias, float eps, const int32_t* rows, const void* scale, const void* shift,
                                     const void* gate, int tab_dt, int act, const void* res, int res_dt, void* out,
                                     int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    int cpl;
    if (row_checks("h3s_norm_mod_act_gate", x_dt, out_dt, C, {x, weight, bias, scale, shift, gate, res, out}, &cpl)) return -1;
    if (!dt_ok(tab_dt) || !dt_ok(res_dt)) return fail("h3s_norm_mod_act_gate: unknown element type");
    if (norm != H3S_NORM_RMS && norm != H3S_NORM_LAYER) return fail("h3s_norm_mod_act_gate: unknown norm");
    if (act != H3S_ACT_NONE && act != H3S_ACT_GELU_TANH && act != H3S_ACT_SILU) return fail("h3s_norm_mod_act_gate: unknown activation");
    Ctx* c = ctx_of(ctx, "h3s_norm_mod_act_gate");
    if (!c) return -1;
#define L3(XDT, CPL, ACT, NORM)                                                                                      \
    norm_mod_act_gate_kernel<XDT, CPL, ACT, NORM><<<grid_rows(M), 256, 0, c->stream>>>(                             \
        x, M, C, weight, bias, eps, rows, scale, shift, gate, tab_dt, res, res_dt, out, out_dt)
#define L2(XDT, CPL, ACT)                                                          \
    if (norm == H3S_NORM_LAYER) L3(XDT, CPL, ACT, H3S_NORM_LAYER);                 \
    else L3(XDT, CPL, ACT, H3S_NORM_RMS)
#define L(XDT, CPL)                                                                \
    if (act == H3S_ACT_GELU_TANH) { L2(XDT, CPL, H3S_ACT_GELU_TANH); }            \
    else if (act == H3S_ACT_SILU) { L2(XDT, CPL, H3S_ACT_SILU); }                 \
    else { L2(XDT, CPL, H3S_ACT_NONE); }
    H3_DT_SWITCH(x_dt, cpl, L)
#undef L
#undef L2
#undef L3
    return launched("h3s_norm_mod_act_gate");
} catch (const std::exception& e) { return fail(e.what()); }

