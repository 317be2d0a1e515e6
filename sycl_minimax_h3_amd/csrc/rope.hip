// rope.hip - h3s_rms_rope (kernels/h3sycl.cpp:1276-1376) and the fused pair h3s_qk_rms_rope: per-head RMS norm and
// the rotary rotation of pairs (j, rot/2 + j), in place.
//
// Layout: a head's D features are D / V 16-byte chunks (V elements of the type), one lane each; a head takes
// CL = pow2ceil(D / V) lanes (the lanes past D / V idle), so a wavefront holds HPW = 64 / CL heads side by side: one
// load or store instruction moves HPW whole heads. With half = rot / 2, feature f = V c + e of the lane's chunk c is
//   f < half:         out_f = n_f cos_f - n_(f + half) sin_f                      (the pair's first value)
//   half <= f < rot:  out_f = n_f cos_(f - half) + n_(f - half) sin_(f - half)   (its second)
//   f >= rot:         out_f = n_f                                                (normalized only)
// with n_f = x_f inv w_f, the reference's arithmetic per element (h3sycl.cpp:1325-1331, 1362-1367). The partner
// values n_(f +- half) come through an LDS area of the wavefront's own: each lane writes its V normalized values,
// then reads its partners' (four at a time when half is a multiple of four, else one by one), so every rot_dim the
// reference takes runs in the same kernel with 16-byte global accesses. The token's (cos, sin) row is staged in LDS
// once a wavefront and each lane takes its elements' pairs from there.
//
// The head's sum of squares is the oracle's canonical sum over CL lanes: each lane adds its chunk's squares in
// order, then an xor butterfly over the head's lanes (offsets CL/2 .. 1).
//
// A token's units (tensor, group of HPW heads) are split over 2^pshift wavefronts, each taking a contiguous share
// of at most 8 units whose loads are all in flight before the first is used. The rows are written back with
// nontemporal stores.
#include "rowcore.h"

namespace h3 {

constexpr int kRopeKU = 8;       // most units a wavefront takes (their loads in flight together)
constexpr int kRopeArea = 512;   // floats of a wavefront's partner area: HPW heads of D <= CL V features

// PURE: every wavefront's share lies inside one tensor (the launch checks it), so a wavefront holds one tensor's
// weights and its units' addresses are one tensor's
template <int XDT, int CL, bool VX, bool PURE>
__global__ __launch_bounds__(256) void rope_kernel(void* x0, void* x1, int64_t M, int H, int D, int64_t stride,
                                                   const float* __restrict__ w0, const float* __restrict__ w1, float eps,
                                                   const float* __restrict__ cs, int rot, int pshift) {
    constexpr int V = Vec<XDT>::V;
    constexpr int ES = 16 / V;                 // bytes an element
    constexpr int HPW = kWave / CL;            // heads side by side in a wavefront
    static_assert(HPW * CL == kWave, "rope_kernel: CL divides 64");
    __shared__ __align__(16) float part_all[4][2][kRopeArea];   // each wavefront's partner areas, by unit parity
    __shared__ __align__(16) float cs_all[4][kRopeArea];        // each wavefront's (cos, sin) row
    const int lane = threadIdx.x & 63, wv = (int) wave_uniform(threadIdx.x >> 6);
    const int64_t wid = (int64_t) blockIdx.x * 4 + wv, tok = wid >> pshift;
    if (tok >= M) return;                       // whole wavefronts: nothing below synchronizes the block
    const int part = (int) (wid & ((1 << pshift) - 1));
    const int half = rot / 2, DC = D / V;
    const int c = lane % CL, hh = lane / CL;
    const bool chunk = c < DC;
    const int f0 = c * V;                       // the lane's first feature inside its head

    // ---- this wavefront's share of the token's units (tensor, group of HPW heads), all uniform ----
    const int ngroups = (H + HPW - 1) / HPW, nunits = (x1 ? 2 : 1) * ngroups;
    const int ubeg = (part * nunits) >> pshift, per = (((part + 1) * nunits) >> pshift) - ubeg;
    const int t0 = ubeg / ngroups, g0 = ubeg - t0 * ngroups;

    // ---- the token's (cos, sin) pairs into LDS, then each element's: cos, and sin signed for its side ----
    float* csl = cs_all[wv];
    const float* ct = cs + tok * (int64_t) rot;               // [half] pairs: rot floats, 8-byte aligned
    for (int i = lane; i < half; i += kWave) *reinterpret_cast<float2*>(csl + 2 * i) = *reinterpret_cast<const float2*>(ct + 2 * i);
    // the weights for this lane's features (pass-through and idle lanes: unused): the share's tensor's, or both
    float wa[2][V];
    if constexpr (PURE) {
        load_f32x((t0 ? w1 : w0) + (chunk ? f0 : 0), wa[0], V);
    } else {
        load_f32x(w0 + (chunk ? f0 : 0), wa[0], V);
        if (x1) load_f32x(w1 + (chunk ? f0 : 0), wa[1], V);
    }
    int pofs[V];                                // the partner's feature (its own for a pass-through element)
    bool pass[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const int f = f0 + e;
        pass[e] = f >= rot;
        pofs[e] = !chunk ? 0 : f < half ? f + half : f < rot ? f - half : f;
    }
    wave_lds_sync();
    float co[V], sg[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const int f = f0 + e, j = f < half ? f : f - half;
        if (!pass[e] && chunk) {
            const float2 t = *reinterpret_cast<const float2*>(csl + 2 * j);
            co[e] = t.x;
            sg[e] = f < half ? -t.y : t.y;
        } else {
            co[e] = 1.0f;
            sg[e] = 0.0f;
        }
    }

    // ---- the units, every load in flight before the first is used. Unit k of the share: tensor tk, group gk (the
    // groups counted on from g0, wrapping into the next tensor); its heads start at a wave-uniform address, and a lane
    // adds its own 32-bit offset. Units past the share read the share's last unit again, and lanes past the heads
    // or the head's chunks read the unit's first chunk: every load is to a valid place and none is branched around;
    // their values are never stored. ----
    const uint32_t lofs = (uint32_t) ((hh * D + f0) * ES);
    auto unit = [&](int k, int& t, int& g) {
        g = g0 + k;
        t = t0;
        if (g >= ngroups) { g -= ngroups; ++t; }
    };
    auto unit_base = [&](int t, int g) {
        return (char*) (t ? x1 : x0) + (tok * stride + (int64_t) g * HPW * D) * ES;
    };
    uint4 raw[kRopeKU];
#pragma unroll
    for (int k = 0; k < kRopeKU; ++k) {
        int t, g;
        unit(k < per ? k : per - 1, t, g);
        const bool ok = chunk && g * HPW + hh < H;
        raw[k] = ld_nt(unit_base(t, g) + (ok ? lofs : 0u));
    }
#pragma unroll
    for (int k = 0; k < kRopeKU; ++k) {
        if (k >= per) break;                    // uniform across the wavefront
        int t, g;
        unit(k, t, g);
        const bool ok = chunk && g * HPW + hh < H;
        float a[V];
        Vec<XDT>::unpack(raw[k], a);
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < V; ++e) s = __builtin_fmaf(a[e], a[e], s);
        s = wave_sum<CL>(ok ? s : 0.0f);
        const float inv = inv_root(s, (float) D, eps);
        float n[V], o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) n[e] = a[e] * inv * (PURE || !t ? wa[0][e] : wa[1][e]);
        if (rot > 0) {
            float* area = part_all[wv][k & 1] + hh * D;
            if (chunk)
#pragma unroll
                for (int e = 0; e < V; e += 4)
                    *reinterpret_cast<float4*>(area + f0 + e) = make_float4(n[e], n[e + 1], n[e + 2], n[e + 3]);
            wave_lds_sync();
            float p[V];
            if constexpr (VX) {
                // half a multiple of 4: each group of four elements has one side and four consecutive partners
#pragma unroll
                for (int e = 0; e < V; e += 4) {
                    const float4 q = *reinterpret_cast<const float4*>(area + pofs[e]);
                    p[e] = q.x; p[e + 1] = q.y; p[e + 2] = q.z; p[e + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) p[e] = area[pofs[e]];
            }
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = pass[e] ? n[e] : n[e] * co[e] + p[e] * sg[e];
        } else {
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = n[e];
        }
        if (ok) st_nt(unit_base(t, g) + lofs, Vec<XDT>::pack(o));
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
    const int CL = pow2ceil((int) (D / V));
    if (D / V > kWave) return fail(std::string(fn) + ": a head of more than 64 16-byte vectors is not supported");
    if (H > (1 << 24)) return fail(std::string(fn) + ": too many heads");
    if (!w0 || (x1 && !w1)) return fail(std::string(fn) + ": the norm weight is required");
    if (rot_dim > 0 && !cs) return fail(std::string(fn) + ": the rotation table is required");
    for (const void* p : {(const void*) x0, (const void*) x1, (const void*) w0, (const void*) w1})
        if (p && !aligned16(p)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    if (cs && ((uintptr_t) cs & 7)) return fail(std::string(fn) + ": the rotation table must be 8-byte aligned");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    // a token's units over the fewest 2^pshift wavefronts that take at most kRopeKU units each (splitting further,
    // each wavefront holding fewer loads, measured slower: 56 heads of 128 at 16896 tokens 105 against 90 us)
    const int64_t nunits = (x1 ? 2 : 1) * ((H + kWave / CL - 1) / (kWave / CL));
    int pshift = 0;
    while ((nunits + (1 << pshift) - 1) >> pshift > kRopeKU) ++pshift;
    if (pshift > 10 || M > (((int64_t) 1 << 31) >> pshift)) return fail(std::string(fn) + ": too many heads a token");
    const bool vx = half % 4 == 0;
    // every wavefront's share inside one tensor: one tensor, or the shares divide each tensor's groups
    const int64_t ngroups = (H + kWave / CL - 1) / (kWave / CL);
    const bool pure = !x1 || (nunits % ((int64_t) 1 << pshift) == 0 && ngroups % (nunits >> pshift) == 0);
    const unsigned grid = (unsigned) (((M << pshift) + 3) / 4);
#define LPV(XDT, CC)                                                                                              \
    {                                                                                                              \
        if (vx && pure) rope_kernel<XDT, CC, true, true><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim, pshift); \
        else if (vx) rope_kernel<XDT, CC, true, false><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim, pshift); \
        else if (pure) rope_kernel<XDT, CC, false, true><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim, pshift); \
        else rope_kernel<XDT, CC, false, false><<<grid, 256, 0, c->stream>>>(x0, x1, M, (int) H, (int) D, stride, w0, w1, eps, cs, rot_dim, pshift); \
    }
#define LD(XDT)                          \
    switch (CL) {                        \
        case 1: LPV(XDT, 1); break;      \
        case 2: LPV(XDT, 2); break;      \
        case 4: LPV(XDT, 4); break;      \
        case 8: LPV(XDT, 8); break;      \
        case 16: LPV(XDT, 16); break;    \
        case 32: LPV(XDT, 32); break;    \
        default: LPV(XDT, 64); break;    \
    }
    switch (x_dt) {
        case H3S_BF16: LD(H3S_BF16); break;
        case H3S_F16: LD(H3S_F16); break;
        default: LD(H3S_F32); break;
    }
#undef LD
#undef LPV
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
