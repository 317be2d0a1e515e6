// quant_impl.h - the row quantizer kernel behind h3s_norm_quant and h3s_int8_linear, instantiated per input type in
// quant_bf16.hip, quant_f16.hip and quant_f32.hip (so the three compile in parallel).
//
// What it computes (the oracle's h3o_norm_quant / h3o_int8_linear quantizer):
//   NORM:  h = round_to_h_dt(x * inv_rms * w [* (1 + scale[t]) + shift[t]])     rms_norm_mod into the reference's
//          scratch h (engine/h3-core/src/dit.rs:340-342, kernels/h3sycl.cpp:766-810)
//   !NORM: h = x                                                               (h3s_int8_linear's own input)
//   y = h . H per group of G features (none, regular h4^(x)k, or Sylvester H2^(x)k; normalized by fl(1/sqrt(G)))
//   s = max(max|y| / 127, 1e-30); q = rint(y / s)                               (kernels/h3sycl.cpp:465-472)
//
// Layout: one 64-wide wavefront per token row. The row is read through 16-byte loads, lane l holding chunks l,
// l + 64, ... (each load instruction of the wave covers 1 KiB of consecutive bytes); the sum of squares is the
// lane's own in chunk order, then an xor butterfly over the 64 lanes (the oracle's canonical order). With a
// rotation, h goes through LDS (as h's bits) so that each lane then owns 64 consecutive features, a "segment": the
// butterfly stages inside a segment run in the lane's registers, and only stages across segments exchange values
// (DPP within a quad / row, LDS crossbar beyond). The codes go back through LDS to the chunk layout, so every global
// store is coalesced as well.
//
// Quantization: q = rint(y / s) with y / s correctly rounded, formed as Markstein's corrected quotient from
// r = fl(1 / s) (one IEEE division per row), then rounded to nearest-even by adding 1.5 * 2^23, whose low byte is
// the two's-complement code. |y / s| <= 127 (1 + 2^-23) for finite y, so the reference's clamp to [-128, 127]
// never binds and is not evaluated.
#pragma once

#include "common.h"

namespace h3 {

constexpr int kSeg = 64;   // features a lane owns in the segment layout
enum { TAB_NONE = 0, TAB_F32 = 1, TAB_BF16 = 2 };

__device__ __forceinline__ float code_of(float y, float s, float r) {
    const float q1 = y * r;
    const float e = __builtin_fmaf(-q1, s, y);
    const float q = __builtin_fmaf(e, r, q1);
    return q + 12582912.0f;                        // 1.5 * 2^23: round to nearest even, the integer in the low bits
}
// the low bytes of four such sums, lowest first
__device__ __forceinline__ uint32_t bytes4(float a, float b, float c, float d) {
    const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0400u);   // a0 b0 0 0
    const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x04000c0cu);   // 0 0 c0 d0
    return lo | hi;
}

// the value of lane (lane ^ OFF): quad permutes, two half-row shifts, a row rotate, a swizzle; beyond, the LDS
// crossbar. No initial value: every lane's source is valid, or (xor 4) overwritten by the second half.
template <int OFF> __device__ __forceinline__ float xl(float v) {
    const int x = __float_as_int(v);
    int r;
    if constexpr (OFF == 1) r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);
    else if constexpr (OFF == 2) r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);
    else if constexpr (OFF == 4) {
        const int t = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0xF, true);      // row_shl:4, right for lanes 0-3, 8-11
        r = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);          // row_shr:4 for lanes 4-7, 12-15
    } else if constexpr (OFF == 8) r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);   // row_ror:8
    else if constexpr (OFF == 16) r = __builtin_amdgcn_ds_swizzle(x, 0x401F);                // xor 16 in 32
    else r = __builtin_amdgcn_ds_bpermute((int) ((__lane_id() ^ (unsigned) OFF) << 2), x);
    return __int_as_float(r);
}
template <int B> __device__ __forceinline__ float quad_lane(float v) {      // lane (lane & ~3) | B
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), B | (B << 2) | (B << 4) | (B << 6), 0xF, 0xF, true));
}

// Sylvester stage across segments: lane ^ OFF pairs; the lower lane forms a + b and the upper a - b, both as
// fma(+-1, own, partner), which is exactly that sum or difference
template <int OFF> __device__ __forceinline__ void syl_cross(float (&v)[kSeg], int lane) {
    const float sg = (lane & OFF) ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < kSeg; ++e) v[e] = __builtin_fmaf(sg, v[e], xl<OFF>(v[e]));
}
// one in-lane Sylvester stage: pairs H apart
template <int H> __device__ __forceinline__ void syl_stage(float (&v)[kSeg]) {
#pragma unroll
    for (int e = 0; e < kSeg; ++e)
        if (!(e & H)) {
            const float a = v[e], b = v[e + H];
            v[e] = a + b;
            v[e + H] = a - b;
        }
}
// one in-lane regular digit: quads D apart
template <int D> __device__ __forceinline__ void reg_digit(float (&v)[kSeg]) {
#pragma unroll
    for (int e = 0; e < kSeg; ++e) {
        if ((e / D) % 4 != 0) continue;
        const float x0 = v[e], x1 = v[e + D], x2 = v[e + 2 * D], x3 = v[e + 3 * D];
        const float t = (x0 + x1) + (x2 + x3);
        v[e] = t - 2.0f * x3; v[e + D] = t - 2.0f * x2; v[e + 2 * D] = t - 2.0f * x1; v[e + 3 * D] = t - 2.0f * x0;
    }
}
// Sylvester stages h = 1, 2, ..., G/2 in order (the oracle's): below 64 inside the lane, then across segments
template <int G> __device__ __forceinline__ void sylvester_seg(float (&v)[kSeg], int lane) {
    if constexpr (G > 1) syl_stage<1>(v);
    if constexpr (G > 2) syl_stage<2>(v);
    if constexpr (G > 4) syl_stage<4>(v);
    if constexpr (G > 8) syl_stage<8>(v);
    if constexpr (G > 16) syl_stage<16>(v);
    if constexpr (G > 32) syl_stage<32>(v);
    if constexpr (G > 64) syl_cross<1>(v, lane);
    if constexpr (G > 128) syl_cross<2>(v, lane);
    if constexpr (G > 256) syl_cross<4>(v, lane);
}
// regular (h4 per base-4 digit, kernels/h3sycl.cpp:433-459): for the four values x0..x3 differing in one digit,
// t = (x0 + x1) + (x2 + x3) (the association of the reference's cross-lane butterfly, h3sycl.cpp:444-453) and
// y_a = t - 2 x_(3-a); digits d = 1, 4, 16 inside the lane, d = 64 (G = 256) across the quad of lanes holding the
// group's four segments: two butterfly adds and the quad mirror (lane a reads lane 3 - a)
template <int G> __device__ __forceinline__ void regular_seg(float (&v)[kSeg], int lane) {
    if constexpr (G > 1) reg_digit<1>(v);
    if constexpr (G > 4) reg_digit<4>(v);
    if constexpr (G > 16) reg_digit<16>(v);
    if constexpr (G > kSeg) {
#pragma unroll
        for (int e = 0; e < kSeg; ++e) {
            const float p = v[e] + xl<1>(v[e]);                  // x0 + x1 (lanes 0, 1), x2 + x3 (lanes 2, 3)
            const float t = p + xl<2>(p);
            const float m = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[e]), 0x1B, 0xF, 0xF, true));   // quad_perm [3,2,1,0]
            v[e] = t - 2.0f * m;
        }
    }
}
// the rotation: for a group size fixed at compile time (GF), a straight-line sequence of stages; otherwise one
// switch on the runtime size (more registers: the cases' allocations add up)
template <int ROT, int GF> __device__ __forceinline__ void rotate_seg(float (&v)[kSeg], int lane, int G) {
    if constexpr (GF != 0) {
        if constexpr (ROT == H3S_ROT_SYLVESTER) sylvester_seg<GF>(v, lane);
        else regular_seg<GF>(v, lane);
    } else if constexpr (ROT == H3S_ROT_SYLVESTER) {
        switch (G) {
            case 2: sylvester_seg<2>(v, lane); break;
            case 4: sylvester_seg<4>(v, lane); break;
            case 8: sylvester_seg<8>(v, lane); break;
            case 16: sylvester_seg<16>(v, lane); break;
            case 32: sylvester_seg<32>(v, lane); break;
            case 64: sylvester_seg<64>(v, lane); break;
            case 128: sylvester_seg<128>(v, lane); break;
            case 256: sylvester_seg<256>(v, lane); break;
            default: sylvester_seg<512>(v, lane); break;
        }
    } else {
        switch (G) {
            case 4: regular_seg<4>(v, lane); break;
            case 16: regular_seg<16>(v, lane); break;
            case 64: regular_seg<64>(v, lane); break;
            default: regular_seg<256>(v, lane); break;
        }
    }
}

// LDS: the row as 16-byte units with a 16-byte pad after each segment's units (segment reads: lanes 144 or 272 bytes
// apart, no bank conflicts); codes: 64 bytes a segment plus 16 of pad
template <int EB> struct Lds {
    static constexpr int UPS = kSeg * EB / 16;
    __device__ static __forceinline__ int unit(int u) { return (u + u / UPS) * 16; }
    static constexpr int bytes_for(int64_t C) { return (int) ((C * EB / 16 + C / kSeg) * 16); }
};

struct QuantArgs {
    const void* x;
    int64_t M, C;
    const float* w;          // NULL: 1
    float eps;
    const int32_t* rows;     // NULL: table row 0
    const void* scale;
    const void* shift;
    int group;
    float cg;                // fl(1 / sqrt(group))
    int8_t* q;
    float* s;
    int lds_bytes;           // per wave
};

template <int XDT, int CPL, int ROT, int HDT, int TAB, bool NORM, int GF = 0>
__global__ __launch_bounds__(256) void quant_kernel(QuantArgs A) {
    constexpr int V = Vec<XDT>::V;
    constexpr int ST = NORM ? HDT : XDT;                     // the type of the values that are quantized
    constexpr int EB = ST == H3S_F32 ? 4 : 2;
    extern __shared__ __attribute__((aligned(16))) char lds_all[];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t row = (int64_t) blockIdx.x * (blockDim.x >> 6) + wv;
    if (row >= A.M) return;
    const int64_t C = A.C, nch = C / V;

    // ---- the row, chunk c = lane + 64 j ----
    uint4 raw[CPL];
    {
        // every lane loads (a chunk past the row's end reads the last one again and is never used): no branch
        // between the loads, so all of them are in flight together
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(A.x) + row * C * (16 / V));
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + (int64_t) kWave * j;
            raw[j] = p[c < nch ? c : nch - 1];
        }
    }
    float v[CPL][V];
    // packed words of the values in ST when they go to LDS as 16-bit (EB == 2)
    uint32_t pk[CPL][V / 2];
#pragma unroll
    for (int j = 0; j < CPL; ++j) Vec<XDT>::unpack(raw[j], v[j]);
    if constexpr (!NORM && EB == 2) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            pk[j][0] = raw[j].x; pk[j][1] = raw[j].y;
            if constexpr (V == 8) { pk[j][2] = raw[j].z; pk[j][3] = raw[j].w; }
        }
    }

    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (lane + (int64_t) kWave * j < nch)
#pragma unroll
                for (int e = 0; e < V; ++e) ss = __builtin_fmaf(v[j][e], v[j][e], ss);
        const float inv = inv_root(wave_sum<kWave>(ss), (float) C, A.eps);
        const int64_t tr = A.rows ? (int64_t) A.rows[row] * C : 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t i = (lane + (int64_t) kWave * j) * V;
            if (i >= C) continue;
            float* o = v[j];
            float wv_[V];
            if (A.w) load_f32x(A.w + i, wv_, V);
            else
#pragma unroll
                for (int e = 0; e < V; ++e) wv_[e] = 1.0f;
#pragma unroll
            for (int e = 0; e < V; ++e) o[e] = o[e] * inv * wv_[e];
            if constexpr (TAB != TAB_NONE) {
                float sc[V], sh[V];
                if constexpr (TAB == TAB_BF16) {
                    load_tab<H3S_BF16>(A.scale, tr + i, sc, V);
                    load_tab<H3S_BF16>(A.shift, tr + i, sh, V);
                } else {
                    load_f32x((const float*) A.scale + tr + i, sc, V);
                    load_f32x((const float*) A.shift + tr + i, sh, V);
                }
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = o[e] * (1.0f + sc[e]) + sh[e];
            }
            // round to h's type, two values a conversion
            if constexpr (HDT != H3S_F32) {
#pragma unroll
                for (int e = 0; e < V; e += 2) {
                    const uint32_t p2 = HDT == H3S_BF16 ? pack_bf16(o[e], o[e + 1]) : pack_f16(o[e], o[e + 1]);
                    pk[j][e / 2] = p2;
                    if constexpr (ROT == H3S_ROT_NONE) {
                        if constexpr (HDT == H3S_BF16) { o[e] = bf16_lo(p2); o[e + 1] = bf16_hi(p2); }
                        else { o[e] = f16_lo(p2); o[e + 1] = f16_hi(p2); }
                    }
                }
            }
        }
    }

    float m = 0.0f;
    int8_t* qrow = A.q + row * C;
    if constexpr (ROT == H3S_ROT_NONE) {
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (lane + (int64_t) kWave * j < nch)
#pragma unroll
                for (int e = 0; e < V; ++e) m = fmaxf(m, fabsf(v[j][e]));
        m = wave_max<kWave>(m);
        const float sc = fmaxf(m / 127.0f, 1e-30f), r = 1.0f / sc;
        if (lane == 0) A.s[row] = sc;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + (int64_t) kWave * j;
            if (c >= nch) continue;
            const float* o = v[j];
            if constexpr (V == 8)
                *reinterpret_cast<uint2*>(qrow + c * 8) =
                    make_uint2(bytes4(code_of(o[0], sc, r), code_of(o[1], sc, r), code_of(o[2], sc, r), code_of(o[3], sc, r)),
                               bytes4(code_of(o[4], sc, r), code_of(o[5], sc, r), code_of(o[6], sc, r), code_of(o[7], sc, r)));
            else
                *reinterpret_cast<uint32_t*>(qrow + c * 4) =
                    bytes4(code_of(o[0], sc, r), code_of(o[1], sc, r), code_of(o[2], sc, r), code_of(o[3], sc, r));
        }
    } else {
        using L = Lds<EB>;
        char* lds = lds_all + wv * A.lds_bytes;
        // ---- chunk layout -> LDS, in ST's bits ----
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + (int64_t) kWave * j;
            if (c >= nch) continue;
            const int64_t e0 = c * V;
            if constexpr (EB == 2) {
                char* a = lds + L::unit((int) (e0 / 8)) + (int) (e0 % 8) * 2;
                if constexpr (V == 8) *reinterpret_cast<uint4*>(a) = make_uint4(pk[j][0], pk[j][1], pk[j][2], pk[j][3]);
                else *reinterpret_cast<uint2*>(a) = make_uint2(pk[j][0], pk[j][1]);
            } else {
#pragma unroll
                for (int k = 0; k < V; k += 4)
                    *reinterpret_cast<float4*>(lds + L::unit((int) ((e0 + k) / 4))) = make_float4(v[j][k], v[j][k + 1], v[j][k + 2], v[j][k + 3]);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // ---- segments: lane l owns features 64 (it 64 + l) .. + 63, it < SI ----
        const int nseg = (int) (C / kSeg);
        constexpr int SI = (CPL * V + kSeg - 1) / kSeg;
        static_assert(SI <= 2, "at most two segment passes");
        // a lane past the row's segments works on a copy of the last one (its results are not used); groups never
        // mix such lanes with real ones (a group's segments are all in the row or all past it)
        auto load_rotate = [&](float (&y)[kSeg], int it) {
            const int sg = it * kWave + lane, sgc = sg < nseg ? sg : nseg - 1;
            if constexpr (EB == 2) {
                uint4 raw_[kSeg / 8];
#pragma unroll
                for (int u = 0; u < kSeg / 8; ++u) raw_[u] = *reinterpret_cast<const uint4*>(lds + L::unit(sgc * (kSeg / 8) + u));
#pragma unroll
                for (int u = 0; u < kSeg / 8; ++u) Vec<ST>::unpack(raw_[u], y + 8 * u);
            } else {
#pragma unroll
                for (int u = 0; u < kSeg / 4; ++u) {
                    const float4 b = *reinterpret_cast<const float4*>(lds + L::unit(sgc * (kSeg / 4) + u));
                    y[4 * u] = b.x; y[4 * u + 1] = b.y; y[4 * u + 2] = b.z; y[4 * u + 3] = b.w;
                }
            }
            rotate_seg<ROT, GF>(y, lane, A.group);
            float mm = 0.0f;
#pragma unroll
            for (int e = 0; e < kSeg; ++e) {
                y[e] = y[e] * A.cg;
                mm = fmaxf(mm, fabsf(y[e]));
            }
            if (sg < nseg) m = fmaxf(m, mm);
        };
        float y0[kSeg], y1[SI > 1 ? kSeg : 1];
        load_rotate(y0, 0);
        if constexpr (SI > 1) load_rotate(y1, 1);
        m = wave_max<kWave>(m);
        const float sc = fmaxf(m / 127.0f, 1e-30f), r = 1.0f / sc;
        if (lane == 0) A.s[row] = sc;
        asm volatile("" ::: "memory");
        // ---- codes: segments -> LDS -> 8-byte pieces of the chunk layout -> global ----
        auto put_codes = [&](const float (&y)[kSeg], int it) {
            const int sg = it * kWave + lane;
            if (sg >= nseg) return;
#pragma unroll
            for (int u = 0; u < kSeg / 16; ++u) {
                const float* yy = y + 16 * u;
                *reinterpret_cast<uint4*>(lds + sg * 80 + 16 * u) =
                    make_uint4(bytes4(code_of(yy[0], sc, r), code_of(yy[1], sc, r), code_of(yy[2], sc, r), code_of(yy[3], sc, r)),
                               bytes4(code_of(yy[4], sc, r), code_of(yy[5], sc, r), code_of(yy[6], sc, r), code_of(yy[7], sc, r)),
                               bytes4(code_of(yy[8], sc, r), code_of(yy[9], sc, r), code_of(yy[10], sc, r), code_of(yy[11], sc, r)),
                               bytes4(code_of(yy[12], sc, r), code_of(yy[13], sc, r), code_of(yy[14], sc, r), code_of(yy[15], sc, r)));
            }
        };
        put_codes(y0, 0);
        if constexpr (SI > 1) put_codes(y1, 1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int64_t npieces = C / 8;                       // piece p (features 8p .. 8p + 7) at 80 (p / 8) + 8 (p % 8)
#pragma unroll
        for (int k = 0; k < (CPL * V) / 8 + 1; ++k) {
            const int64_t p = lane + (int64_t) kWave * k;
            if (p < npieces) *reinterpret_cast<uint2*>(qrow + p * 8) = *reinterpret_cast<const uint2*>(lds + (p / 8) * 80 + (p % 8) * 8);
        }
    }
}

// Launches the kernel for one input type. Checks shapes it cannot take.
template <int XDT>
int quant_launch(Ctx* c, const char* fn, QuantArgs A, int rot, int hdt, int tab, bool norm) {
    constexpr int V = Vec<XDT>::V;
    const int64_t per_lane = (A.C / V + kWave - 1) / kWave;
    const int cpl = per_lane <= 2 ? 2 : per_lane <= 8 ? 8 : per_lane <= 16 ? 16 : 0;
    if (!cpl)
        return fail(std::string(fn) + ": rows longer than 16 x 64 16-byte vectors (8192 16-bit or 4096 float32 features) are not supported");
    const int st = norm ? hdt : XDT;
    const int eb = st == H3S_F32 ? 4 : 2;
    A.lds_bytes = rot == H3S_ROT_NONE ? 0 : (eb == 2 ? Lds<2>::bytes_for(A.C) : Lds<4>::bytes_for(A.C));
    int wpb = 4;                                          // waves a block, within 64 KiB of LDS
    while (wpb > 1 && (size_t) A.lds_bytes * wpb > 64 * 1024) wpb /= 2;
    if ((size_t) A.lds_bytes * wpb > 64 * 1024) return fail(std::string(fn) + ": a rotated row of this length does not fit the LDS");
    const unsigned grid = (unsigned) ((A.M + wpb - 1) / wpb);
    const size_t shm = (size_t) A.lds_bytes * wpb;
#define QK(CPL, ROT, HDT, TAB, NRM) quant_kernel<XDT, CPL, ROT, HDT, TAB, NRM><<<grid, 64 * wpb, shm, c->stream>>>(A)
#define QF(CPL, ROT, TAB, G) quant_kernel<XDT, CPL, ROT, XDT, TAB, true, G><<<grid, 64 * wpb, shm, c->stream>>>(A)
    // compile-time group sizes for the common cases: 16-bit x and h of the same type, CPL 8 or 16
    if constexpr (XDT != H3S_F32) {
        const bool syl = rot == H3S_ROT_SYLVESTER && (A.group == 64 || A.group == 128 || A.group == 256);
        const bool reg = rot == H3S_ROT_REGULAR && A.group == 256;
        if (norm && hdt == XDT && (cpl == 8 || cpl == 16) && (syl || reg)) {
#define QFG(CPL, TAB)                                                              \
    if (reg) QF(CPL, H3S_ROT_REGULAR, TAB, 256);                                   \
    else if (A.group == 64) QF(CPL, H3S_ROT_SYLVESTER, TAB, 64);                   \
    else if (A.group == 128) QF(CPL, H3S_ROT_SYLVESTER, TAB, 128);                 \
    else QF(CPL, H3S_ROT_SYLVESTER, TAB, 256);
#define QFT(CPL)                                          \
    if (tab == TAB_BF16) { QFG(CPL, TAB_BF16) }           \
    else if (tab == TAB_F32) { QFG(CPL, TAB_F32) }        \
    else { QFG(CPL, TAB_NONE) }
            if (cpl == 8) { QFT(8) }
            else { QFT(16) }
#undef QFT
#undef QFG
            return launched(fn);
        }
        if (!norm && reg && (cpl == 8 || cpl == 16)) {
            if (cpl == 8) quant_kernel<XDT, 8, H3S_ROT_REGULAR, H3S_F32, TAB_NONE, false, 256><<<grid, 64 * wpb, shm, c->stream>>>(A);
            else quant_kernel<XDT, 16, H3S_ROT_REGULAR, H3S_F32, TAB_NONE, false, 256><<<grid, 64 * wpb, shm, c->stream>>>(A);
            return launched(fn);
        }
    }
#define QT(CPL, ROT, HDT)                                          \
    if (tab == TAB_BF16) QK(CPL, ROT, HDT, TAB_BF16, true);        \
    else if (tab == TAB_F32) QK(CPL, ROT, HDT, TAB_F32, true);     \
    else QK(CPL, ROT, HDT, TAB_NONE, true)
#define QH(CPL, ROT)                                       \
    if (hdt == H3S_BF16) { QT(CPL, ROT, H3S_BF16); }       \
    else if (hdt == H3S_F16) { QT(CPL, ROT, H3S_F16); }    \
    else { QT(CPL, ROT, H3S_F32); }
#define QR(CPL)                                                                                   \
    if (norm) {                                                                                   \
        if (rot == H3S_ROT_SYLVESTER) { QH(CPL, H3S_ROT_SYLVESTER) }                               \
        else if (rot == H3S_ROT_REGULAR) { QH(CPL, H3S_ROT_REGULAR) }                              \
        else { QH(CPL, H3S_ROT_NONE) }                                                             \
    } else {                                                                                      \
        if (rot == H3S_ROT_REGULAR) QK(CPL, H3S_ROT_REGULAR, H3S_F32, TAB_NONE, false);           \
        else QK(CPL, H3S_ROT_NONE, H3S_F32, TAB_NONE, false);                                     \
    }
    if (cpl == 2) { QR(2) }
    else if (cpl == 8) { QR(8) }
    else { QR(16) }
#undef QR
#undef QH
#undef QT
#undef QF
#undef QK
    return launched(fn);
}

}  // namespace h3
