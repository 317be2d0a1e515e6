// rope.hip - h3s_rms_rope (kernels/h3sycl.cpp:1276-1376) and the fused pair h3s_qk_rms_rope: per-head RMS norm and
// the rotary rotation of pairs (j, rot/2 + j), in place, q and k of a token in one wave.
//
// A head's D features are dealt to "slots", one lane each. With V the elements of a 16-byte vector and
// half = rot / 2, rotated slot p takes the pairs j in [pV, min(pV + V, half)) - the lane owns both values of each of
// its pairs, so the rotation needs no exchange - and pass-through slot q the features [rot + qV, min(rot + qV + V,
// D)). A head takes P2 lanes (its slot count rounded up to a power of two), so a wave holds 64 / P2 heads side by
// side; the head's sum of squares is the lane's own (its first features, then their partners), then an xor
// butterfly over its P2 lanes: the canonical order of the CPU oracle. One wave per token, or two that take half its
// (tensor, head group) units each: a wave reads the token's cos/sin row and the weights once, then its heads. Two
// kernels:
//   rope_kernel      half and D - rot whole 16-byte vectors (rot = D, 96 or 48 at D = 128, the VAE's 48 at 64):
//                    a slot is whole chunks, read and written straight from and to memory with 16-byte accesses;
//   rope_any_kernel  any even rot (the DiT's rot = 6 x its frequencies, e.g. 126 for 21): a head is copied to
//                    LDS in 16-byte chunks, each slot reads its features from there one by one, writes its results
//                    back, and the head goes out in 16-byte chunks.
// The rows are written back with nontemporal stores.
#include "rowcore.h"

namespace h3 {

constexpr int kUnits = 8;   // (tensor, head group) units whose loads are in flight together
constexpr int kRopeMaxD = 1024;   // the largest head rope_kernel takes: 64 slots of V pairs (16-bit types)

// PARTS: wavefronts a token (2: each takes half its (tensor, head group) units); KU: units whose loads are in
// flight together
template <int XDT, int P2, int PARTS, int KU = kUnits / PARTS>
__global__ __launch_bounds__(256) void rope_kernel(void* x0, void* x1, int64_t M, int H, int D, int64_t stride,
                                                   const float* __restrict__ w0, const float* __restrict__ w1, float eps,
                                                   const float* __restrict__ cs, int rot) {
    constexpr int V = Vec<XDT>::V;
    constexpr int HPW = kWave / P2;   // heads side by side in a wave
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6), tok = wid / PARTS;
    const int part = (int) (wid - tok * PARTS);
    const int half = rot / 2, nrot = half / V, npass = (D - rot) / V, P = nrot + npass;
    const int slot = lane % P2, hh = lane / P2;
    const bool active = slot < P, rotated = slot < nrot;
    // the token's cos/sin pairs of this lane's slot, in flight during the weights' staging below and taken apart
    // only where the rotation uses them
    float4 csv[V / 2];
    if (rotated && tok < M) {
        const float* c = cs + (tok * half + (int64_t) slot * V) * 2;
#pragma unroll
        for (int k = 0; k < V / 2; ++k) csv[k] = *reinterpret_cast<const float4*>(c + 4 * k);
    }
    // the norm weights of both tensors, staged once a block (every thread, before any wavefront leaves): read
    // from global memory after each unit's reduction, their wait also waited for the batch's remaining rows
    __shared__ __attribute__((aligned(16))) float wl[2][kRopeMaxD];
    for (int i = threadIdx.x; i < D; i += 256) {
        wl[0][i] = w0[i];
        if (x1) wl[1][i] = w1[i];
    }
    __syncthreads();
    if (tok >= M) return;
    const int off0 = rotated ? slot * V : rot + (slot - nrot) * V;   // this lane's chunk(s) inside the head
    const int off1 = half + slot * V;

    const int ngroups = (H + HPW - 1) / HPW;
    const int ntens = x1 ? 2 : 1;
    const int per = ntens * ngroups / PARTS, ubeg = part * per, uend = ubeg + per;   // this wavefront's units
    for (int u0 = ubeg; u0 < uend; u0 += KU) {
        uint4 ra[KU], rb[KU];
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            // every lane loads from a valid place (idle lanes and units past the end read head 0 / the last unit
            // again, and their values are never used): no branch between the loads
            const int u = u0 + k < uend ? u0 + k : uend - 1, t = u / ngroups, h0 = (u % ngroups) * HPW + hh;
            const int head = active && h0 < H ? h0 : 0;
            const uint16_t* base = (const uint16_t*) (t ? x1 : x0) + (tok * stride + (int64_t) head * D) * (16 / V / 2);
            ra[k] = ld_nt(base + (active ? off0 : 0) * (16 / V / 2));
            rb[k] = ld_nt(base + (rotated ? off1 : 0) * (16 / V / 2));
        }
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int u = u0 + k;
            if (u >= uend) break;     // uniform across the wave
            const int t = u / ngroups, head = (u % ngroups) * HPW + hh;
            const bool ok = active && head < H;
            float a[V], b[V];
            Vec<XDT>::unpack(ra[k], a);
            Vec<XDT>::unpack(rb[k], b);
            float s = 0.0f;
            if (ok) {
#pragma unroll
                for (int e = 0; e < V; ++e) s = __builtin_fmaf(a[e], a[e], s);
                if (rotated)
#pragma unroll
                    for (int e = 0; e < V; ++e) s = __builtin_fmaf(b[e], b[e], s);
            }
            s = wave_sum<P2>(s);
            if (!ok) continue;
            const float inv = inv_root(s, (float) D, eps);
            const float* w = wl[t];
            float wa[V];
            load_f32x(w + off0, wa, V);
            uint16_t* base = (uint16_t*) (t ? x1 : x0) + (tok * stride + (int64_t) head * D) * (16 / V / 2);
            if (rotated) {
                float wb[V], oa[V], ob[V], co[V], si[V];
                load_f32x(w + off1, wb, V);
#pragma unroll
                for (int k = 0; k < V / 2; ++k) {
                    co[2 * k] = csv[k].x; si[2 * k] = csv[k].y; co[2 * k + 1] = csv[k].z; si[2 * k + 1] = csv[k].w;
                }
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float A = a[e] * inv * wa[e], B = b[e] * inv * wb[e];
                    oa[e] = A * co[e] - B * si[e];
                    ob[e] = B * co[e] + A * si[e];
                }
                st_nt(base + off0 * (16 / V / 2), Vec<XDT>::pack(oa));
                st_nt(base + off1 * (16 / V / 2), Vec<XDT>::pack(ob));
            } else {
                float oa[V];
#pragma unroll
                for (int e = 0; e < V; ++e) oa[e] = a[e] * inv * wa[e];
                st_nt(base + off0 * (16 / V / 2), Vec<XDT>::pack(oa));
            }
        }
    }
}

// A wavefront's LDS staging area is its own, so wave_lds_sync (common.h), not a workgroup barrier, orders it.

constexpr int kAnyStage = 2048;   // bytes of LDS a wavefront stages: 64 / P2 heads of D <= 2 P2 V elements

template <int XDT, int P2>
__global__ __launch_bounds__(256) void rope_any_kernel(void* x0, void* x1, int64_t M, int H, int D, int64_t stride,
                                                       const float* __restrict__ w0, const float* __restrict__ w1,
                                                       float eps, const float* __restrict__ cs, int rot) {
    constexpr int V = Vec<XDT>::V;
    constexpr int ES = 16 / V;        // bytes an element
    constexpr int HPW = kWave / P2;   // heads side by side in a wave
    __shared__ __align__(16) char stage_all[4][kAnyStage];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t tok = (int64_t) blockIdx.x * 4 + wv;
    if (tok >= M) return;
    char* stage = stage_all[wv];
    const int half = rot / 2, nrot = (half + V - 1) / V, npass = (D - rot + V - 1) / V, P = nrot + npass;
    const int slot = lane % P2, hh = lane / P2;
    const bool rotated = slot < nrot, active = slot < P;
    // this slot's first feature and how many it has (for a rotated slot: its pairs; their partners are half on)
    const int f0 = rotated ? slot * V : rot + (slot - nrot) * V;
    const int n = !active ? 0 : rotated ? min(V, half - f0) : min(V, D - f0);
    float co[V], si[V], wa[2][V], wb[2][V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
        co[e] = 1.0f; si[e] = 0.0f;
        wa[0][e] = wa[1][e] = wb[0][e] = wb[1][e] = 0.0f;
        if (e < n) {
            wa[0][e] = w0[f0 + e];
            if (x1) wa[1][e] = w1[f0 + e];
            if (rotated) {
                const float2 t = *reinterpret_cast<const float2*>(cs + (tok * half + f0 + e) * 2);
                co[e] = t.x; si[e] = t.y;
                wb[0][e] = w0[half + f0 + e];
                if (x1) wb[1][e] = w1[half + f0 + e];
            }
        }
    }
    auto get = [&](int e) -> float {                          // element e of this lane's head, from the stage
        if constexpr (XDT == H3S_F32) return reinterpret_cast<const float*>(stage)[hh * D + e];
        else {
            const uint32_t b = reinterpret_cast<const uint16_t*>(stage)[hh * D + e];
            return XDT == H3S_BF16 ? bf16_lo(b) : f16_lo(b);
        }
    };
    auto put = [&](int e, float v) {                          // v rounded to the element type, into the stage
        if constexpr (XDT == H3S_F32) reinterpret_cast<float*>(stage)[hh * D + e] = v;
        else reinterpret_cast<uint16_t*>(stage)[hh * D + e] =
                 (uint16_t) (XDT == H3S_BF16 ? pack_bf16(v, 0.0f) : pack_f16(v, 0.0f));
    };
    const int DC = D / V;                                     // chunks a head; a lane copies chunks slot + P2 i
    const int ngroups = (H + HPW - 1) / HPW, ntens = x1 ? 2 : 1, nunits = ntens * ngroups;
    // the head of unit u this lane's group copies, as a chunk pointer (NULL past the last head)
    auto head_of = [&](int u) -> uint4* {
        const int t = u / ngroups, h = (u % ngroups) * HPW + hh;
        if (h >= H) return nullptr;
        return reinterpret_cast<uint4*>((char*) (t ? x1 : x0) + (tok * stride + (int64_t) h * D) * ES);
    };
    uint4 buf[2];
    auto fetch = [&](int u) {
        const uint4* hp = head_of(u);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = slot + P2 * i;
            if (hp && c < DC) buf[i] = ld_nt(hp + c);
        }
    };
    fetch(0);
    for (int u = 0; u < nunits; ++u) {
        uint4* hp = head_of(u);
        const int t = u / ngroups;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = slot + P2 * i;
            if (hp && c < DC) *reinterpret_cast<uint4*>(stage + (hh * D + c * V) * ES) = buf[i];
        }
        if (u + 1 < nunits) fetch(u + 1);                     // the next unit's chunks in flight meanwhile
        wave_lds_sync();
        float a[V], b[V];
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            a[e] = b[e] = 0.0f;
            if (hp && e < n) { a[e] = get(f0 + e); s = __builtin_fmaf(a[e], a[e], s); }
        }
        if (rotated)
#pragma unroll
            for (int e = 0; e < V; ++e)
                if (hp && e < n) { b[e] = get(half + f0 + e); s = __builtin_fmaf(b[e], b[e], s); }
        s = wave_sum<P2>(s);
        const float inv = inv_root(s, (float) D, eps);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            if (!hp || e >= n) continue;
            const float A = a[e] * inv * (t ? wa[1][e] : wa[0][e]);
            if (rotated) {
                const float B = b[e] * inv * (t ? wb[1][e] : wb[0][e]);
                put(f0 + e, A * co[e] - B * si[e]);
                put(half + f0 + e, B * co[e] + A * si[e]);
            } else {
                put(f0 + e, A);
            }
        }
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = slot + P2 * i;
            if (hp && c < DC) st_nt(hp + c, *reinterpret_cast<const uint4*>(stage + (hh * D + c * V) * ES));
        }
        wave_lds_sync();                                      // the stage is read before the next unit fills it
    }
}

static int pow2ceil(int n) { int p = 1; while (p < n) p *= 2; return p; }

static int rope_launch(const char* fn, void* ctx, void* x0, void* x1, int x_dt, int64_t M, int64_t H, int64_t D,
                       int64_t stride, const float* w0, const float* w1, float eps, const float* cs, int rot_dim) {
    if (M <= 0 || H <= 0 || D <= 0) return 0;
    if (rot_dim < 0 || rot_dim > D || rot_dim % 2 != 0 || (D - rot_dim) % 2 != 0)
        return fail(std::string(fn) + ": rot_dim must be even, at most D, and leave an even remainder");
    if (stride < H * D) return fail(std::string(fn) + ": the row stride is shorter than a row");
    if (!dt_ok(x_dt)) return fail(std::string(fn) + ": unknown element type");
    const int V = vec_of(x_dt);
    const int64_t half = rot_dim / 2;
    if (D % V != 0 || stride % V != 0)
        return fail(std::string(fn) + ": D and the stride must be whole 16-byte vectors (multiples of " + std::to_string(V) + ")");
    const int P = (int) ((half + V - 1) / V + (D - rot_dim + V - 1) / V);
    const int P2 = pow2ceil(P);
    if (P2 > kWave || D > kRopeMaxD) return fail(std::string(fn) + ": a head of more than 64 slots is not supported");
    if (H > (1 << 24)) return fail(std::string(fn) + ": too many heads");
    if (!w0 || (x1 && !w1)) return fail(std::string(fn) + ": the norm weight is required");
    if (rot_dim > 0 && !cs) return fail(std::string(fn) + ": the rotation table is required");
    for (const void* p : {(const void*) x0, (const void*) x1, (const void*) w0, (const void*) w1, (const void*) cs})
        if (p && !aligned16(p)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    // whole-chunk slots go straight through memory; any other split through the wavefront's LDS stage
    const bool whole = half % V == 0 && (D - rot_dim) % V == 0;
    // a token's units (tensor, group of 64 / P2 heads) in two wavefronts where they split evenly (whole-chunk
    // slots): twice the wavefronts, each holding half the loads, so the last of them end sooner
    const int64_t nunits = (x1 ? 2 : 1) * ((H + kWave / P2 - 1) / (kWave / P2));
    const int parts = whole && nunits % 2 == 0 ? 2 : 1;
    const unsigned grid = (unsigned) ((M * parts + 3) / 4);
#define LP(XDT, PP)                                                                                               \
    if (whole && parts == 2)                                                                                      \
        rope_kernel<XDT, PP, 2><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim); \
    else if (whole)                                                                                               \
        rope_kernel<XDT, PP, 1><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim); \
    else rope_any_kernel<XDT, PP><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim)
#define LD(XDT)                         \
    switch (P2) {                       \
        case 1: LP(XDT, 1); break;      \
        case 2: LP(XDT, 2); break;      \
        case 4: LP(XDT, 4); break;      \
        case 8: LP(XDT, 8); break;      \
        case 16: LP(XDT, 16); break;    \
        case 32: LP(XDT, 32); break;    \
        default: LP(XDT, 64); break;    \
    }
    switch (x_dt) {
        case H3S_BF16: LD(H3S_BF16); break;
        case H3S_F16: LD(H3S_F16); break;
        default: LD(H3S_F32); break;
    }
#undef LD
#undef LP
    return launched(fn);
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_rms_rope(void* ctx, void* x, int x_dt, int64_t M, int64_t H, int64_t D, int64_t stride, const float* weight,
                            float eps, const float* cs, int rot_dim) try {
    return rope_launch("h3s_rms_rope", ctx, x, nullptr, x_dt, M, H, D, stride, weight, nullptr, eps, cs, rot_dim);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_qk_rms_rope(void* ctx, void* q, void* k, int x_dt, int64_t M, int64_t H, int64_t D, int64_t stride,
                               const float* wq, const float* wk, float eps, const float* cs, int rot_dim) try {
    if (!q || !k) return fail("h3s_qk_rms_rope: q and k are required");
    return rope_launch("h3s_qk_rms_rope", ctx, q, k, x_dt, M, H, D, stride, wq, wk, eps, cs, rot_dim);
} catch (const std::exception& e) { return fail(e.what()); }
