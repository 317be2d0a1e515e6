// quant_impl.h - the row quantizer kernel behind h3s_norm_quant and h3s_int8_linear, instantiated per input type in
// quant_bf16.hip, quant_f16.hip and quant_f32.hip.
//
// What it computes (the oracle's h3o_norm_quant / h3o_int8_linear quantizer / h3o_swiglu_quant):
//   NORM:   h = round_to_h_dt(x * inv_rms [* w] [* (1 + scale[t]) + shift[t]])  rms_norm_mod into the reference's
//           scratch h (engine/h3-core/src/dit.rs:340-342, kernels/h3sycl.cpp:766-810)
//   RAW:    h = x                                                               (h3s_int8_linear's own input)
//   SWIGLU: h = round_to_h_dt(silu(g) * u), x = [g | u] rows of 2C              (h3s_swiglu into the MLP's scratch
//           act, then fc2's quantizer: engine/h3-core/src/dit.rs:363-364, kernels/h3sycl.cpp:1378-1419)
//   y = h . H per group of G features (none, regular h4^(x)k, or Sylvester H2^(x)k), then * fl(1/sqrt(G))
//   s = max(max|y| / 127, 1e-30); q = rint(y / s)                               (kernels/h3sycl.cpp:465-472)
//
// Layout: rowcore.h's. A rotation group of G features is G/V consecutive chunks, so it lives in G/V consecutive
// lanes (G/V <= 64: one wavefront) at the same chunk slot of each: its butterfly stages inside a chunk run in the
// lane's registers, and the stages across chunks exchange values between lanes (DPP inside a row of 16 lanes, the
// LDS crossbar beyond), with no staging through memory. A group's chunks are all inside the row or all past it, so
// lanes that hold a clamped copy of the last chunk only ever exchange with each other. The group size is a runtime
// value: each possible stage is compiled once and runs when the group is large enough.
//
// Quantization: q = rint(y / s) with y / s correctly rounded, formed as Markstein's corrected quotient from
// r = fl(1 / s) (one IEEE division per row), then rounded to nearest-even by adding 1.5 * 2^23, whose low byte is
// the two's-complement code. |y / s| <= 127 (1 + 2^-23) for finite y, so the reference's clamp to [-128, 127]
// never binds and is not evaluated.
#pragma once

#include "rowcore.h"

namespace h3 {

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

// the value held by lane (lane ^ X) of the wavefront: quad permutes (1, 2, 3), two half-row shifts (4), a row
// rotate (8), a swizzle inside each half of the wave (other X < 32), the LDS crossbar (X >= 32)
template <int X> __device__ __forceinline__ float lane_xor(float v) {
    static_assert(X > 0 && X < 64, "lane_xor: 1 .. 63");
    const int x = __float_as_int(v);
    int r;
    if constexpr (X == 1) r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);          // quad_perm [1,0,3,2]
    else if constexpr (X == 2) r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);     // quad_perm [2,3,0,1]
    else if constexpr (X == 3) r = __builtin_amdgcn_mov_dpp(x, 0x1B, 0xF, 0xF, true);     // quad_perm [3,2,1,0]
    else if constexpr (X == 4) {
        const int t = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0xF, true);                  // row_shl:4, lanes 0-3, 8-11
        r = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);                      // row_shr:4, lanes 4-7, 12-15
    } else if constexpr (X == 8) r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);  // row_ror:8
    else if constexpr (X < 32) r = __builtin_amdgcn_ds_swizzle(x, 0x1F | (X << 10));      // and 0x1f, xor X
    else r = __builtin_amdgcn_ds_bpermute((int) ((__lane_id() ^ (unsigned) X) << 2), x);
    return __int_as_float(r);
}

// ---- Sylvester: stages h = 1, 2, ..., G/2 in order, (a, b) -> (a + b, a - b) for the pair h apart ----
template <int V, int H> __device__ __forceinline__ void syl_in(float (&v)[V]) {
#pragma unroll
    for (int e = 0; e < V; ++e)
        if (!(e & H)) {
            const float a = v[e], b = v[e + H];
            v[e] = a + b;
            v[e + H] = a - b;
        }
}
// The stages across lanes keep each lane's values up to a sign fixed by the lane: at the stage S chunks apart the
// lower chunk forms own + partner and the upper chunk own - partner, which is the negation of the a - b it owes.
// Both partners carry the same sign from the earlier stages (they differ only in chunk bit S), and rounding to
// nearest is symmetric, so every value stays exactly +-(the value of the plain butterfly); the sign is
// (-1)^popcount(pos & (G/V - 1)) for the lane's chunk position pos in its group, folded into the final multiply by
// fl(1/sqrt(G)). One fused multiply-add with the partner's value taken straight from a neighbouring lane
// (own + partner * (+-1)) per value and stage.
// Chunk positions: in the plain layout (SW false) lane l holds position l of its run of 16 lanes, so the partner S
// chunks away is lane l ^ S. In the swapped layout (SW true) lane l holds position swap3(l) = l ^ 3 bit2(l), an
// involution that leaves the partners 1, 2, 8, 16 and 32 chunks away at lanes l ^ 1, l ^ 2, l ^ 8, l ^ 16 and
// l ^ 32, and moves the partner 4 chunks away to lane l ^ 7, which DPP's row_half_mirror reaches in one instruction
// (l ^ 4 takes two).
// For partners 1, 2 or 8 lanes away (and 7 in the swapped layout) the partner's value comes through the DPP operand
// of v_fmac_f32 itself (one instruction a value); s_nop 1 gives the two wait states a DPP read needs after the VALU
// write of the previous stage.
__device__ __forceinline__ int swap3(int l) { return l ^ (((l >> 2) & 1) * 3); }
#define H3_FMAC_DPP8(CTRL, SRC)                                                                                 \
    asm volatile("s_nop 1\n"                                                                                    \
                 "v_fmac_f32_dpp %0, %8, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                             \
                 "v_fmac_f32_dpp %1, %9, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                             \
                 "v_fmac_f32_dpp %2, %10, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
                 "v_fmac_f32_dpp %3, %11, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
                 "v_fmac_f32_dpp %4, %12, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
                 "v_fmac_f32_dpp %5, %13, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
                 "v_fmac_f32_dpp %6, %14, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
                 "v_fmac_f32_dpp %7, %15, %16 " CTRL " row_mask:0xf bank_mask:0xf"                               \
                 : "=v"(o[0]), "=v"(o[1]), "=v"(o[2]), "=v"(o[3]), "=v"(o[4]), "=v"(o[5]), "=v"(o[6]), "=v"(o[7]) \
                 : "v"(SRC[0]), "v"(SRC[1]), "v"(SRC[2]), "v"(SRC[3]), "v"(SRC[4]), "v"(SRC[5]), "v"(SRC[6]),      \
                   "v"(SRC[7]), "v"(sg), "0"(v[0]), "1"(v[1]), "2"(v[2]), "3"(v[3]), "4"(v[4]), "5"(v[5]),       \
                   "6"(v[6]), "7"(v[7]))
template <int V, int S, bool SW> __device__ __forceinline__ void syl_x(float (&v)[V], int pos) {
    static_assert(!SW || V == 8, "syl_x: the swapped layout has 8 values a chunk");
    const float sg = (pos & S) ? -1.0f : 1.0f;
    if constexpr (V == 8 && (S == 1 || S == 2 || S == 8 || (S == 4 && SW))) {
        float o[8];
        if constexpr (S == 1) H3_FMAC_DPP8("quad_perm:[1,0,3,2]", v);
        else if constexpr (S == 2) H3_FMAC_DPP8("quad_perm:[2,3,0,1]", v);
        else if constexpr (S == 4) H3_FMAC_DPP8("row_half_mirror", v);
        else H3_FMAC_DPP8("row_ror:8", v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = o[e];
    } else if constexpr (V == 8 && S == 4) {
        // lane ^ 4 = (lane ^ 3) ^ 7: a quad reversal, then the half-row mirror inside the multiply-add
        float x[8], o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[e]), 0x1B, 0xF, 0xF, true));
        H3_FMAC_DPP8("row_half_mirror", x);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = o[e];
    } else {
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = __builtin_fmaf(lane_xor<S>(v[e]), sg, v[e]);
    }
}
#undef H3_FMAC_DPP8
// the sign the cross-lane stages leave on the values of the chunk at position pos
template <int V> __device__ __forceinline__ float syl_sign(int pos, int G) {
    const int span = G / V;                               // lanes of a group (1 when the group is inside a chunk)
    return span > 1 && (__builtin_popcount((unsigned) (pos & (span - 1))) & 1) ? -1.0f : 1.0f;
}
template <int V, bool SW = false> __device__ __forceinline__ void sylvester(float (&v)[V], int pos, int G) {
    if (G > 1) syl_in<V, 1>(v);
    if (G > 2) syl_in<V, 2>(v);
    if constexpr (V == 8)
        if (G > 4) syl_in<V, 4>(v);
    if (G > V) syl_x<V, 1, SW>(v, pos);
    if (G > 2 * V) syl_x<V, 2, SW>(v, pos);
    if (G > 4 * V) syl_x<V, 4, SW>(v, pos);
    if (G > 8 * V) syl_x<V, 8, SW>(v, pos);
    if (G > 16 * V) syl_x<V, 16, SW>(v, pos);
    if (G > 32 * V) syl_x<V, 32, SW>(v, pos);
}

// ---- regular: one base-4 digit at a time, low digit first (kernels/h3sycl.cpp:433-456); for the four values
// x0..x3 that differ in that digit, y_a = t - 2 x_(3-a). t is formed as the reference's group-of-256 kernel forms
// it: the digits of stride 1 and 4 (inside its work-item's registers) left to right, ((x0 + x1) + x2) + x3
// (h3sycl.cpp:440); the digits of stride 16 and 64 (across its lanes) pairwise, (x0 + x1) + (x2 + x3)
// (h3sycl.cpp:452-453). Float addition commutes bit for bit, so every lane forms the same t from its own view. ----
// the value of lane 4 (lane / 4) + p[lane % 4] of each quad, for the DPP quad_perm control CTRL
template <int CTRL> __device__ __forceinline__ float quad(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// the digit of stride 1, inside a chunk; t - 2 x as one fma (2 x is exact below 2^127, so this is the value of
// t - 2.0f * x; the digits across lanes keep the two instructions, whose partner values come through DPP)
template <int V> __device__ __forceinline__ void reg_in(float (&v)[V]) {
#pragma unroll
    for (int e = 0; e < V; e += 4) {
        const float x0 = v[e], x1 = v[e + 1], x2 = v[e + 2], x3 = v[e + 3];
        const float t = ((x0 + x1) + x2) + x3;
        v[e] = __builtin_fmaf(-2.0f, x3, t); v[e + 1] = __builtin_fmaf(-2.0f, x2, t);
        v[e + 2] = __builtin_fmaf(-2.0f, x1, t); v[e + 3] = __builtin_fmaf(-2.0f, x0, t);
    }
}
// the digit of stride 4 with V = 8: x0, x1 at e and e + 4 of an even lane, x2, x3 at e and e + 4 of the odd lane
// beside it. The even lane's pair sum x0 + x1 goes to both lanes (quad_perm [0,0,2,2]), then the odd lane's x2 and
// x3 are added in turn ([1,1,3,3]); the mirror x_(3-a) is the partner's value at the other half of the chunk
// ([1,0,3,2]).
__device__ __forceinline__ void reg_pair(float (&v)[8]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float lo = v[r], hi = v[r + 4];
        const float t = (quad<0xA0>(lo + hi) + quad<0xF5>(lo)) + quad<0xF5>(hi);
        v[r] = t - 2.0f * quad<0xB1>(hi);
        v[r + 4] = t - 2.0f * quad<0xB1>(lo);
    }
}
// the digit of stride 4 with V = 4: x0..x3 in the four lanes of a quad, taken in order (quad_perm [a,a,a,a]); the
// mirror from the reversed quad ([3,2,1,0])
__device__ __forceinline__ void reg_quad(float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float t = ((quad<0x00>(v[e]) + quad<0x55>(v[e])) + quad<0xAA>(v[e])) + quad<0xFF>(v[e]);
        v[e] = t - 2.0f * quad<0x1B>(v[e]);
    }
}
// the digit whose four values sit in lanes S apart (a = (lane / S) % 4): the own pair x_a + x_(a^1), the other pair
// from the lanes 2S away, and the mirror x_(3-a) from the lane 3S away
template <int V, int S> __device__ __forceinline__ void reg_x(float (&v)[V]) {
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const float pv = v[e] + lane_xor<S>(v[e]);
        const float t = pv + lane_xor<2 * S>(pv);
        v[e] = t - 2.0f * lane_xor<3 * S>(v[e]);
    }
}
template <int V> __device__ __forceinline__ void regular(float (&v)[V], int G) {
    if (G > 1) reg_in<V>(v);
    if constexpr (V == 8) {
        if (G > 4) reg_pair(v);
        if (G > 16) reg_x<8, 2>(v);
        if (G > 64) reg_x<8, 8>(v);
    } else {
        if (G > 4) reg_quad(v);
        if (G > 16) reg_x<4, 4>(v);
        if (G > 64) reg_x<4, 16>(v);
    }
}

// A kernel's ROT template value: the rotation kind (H3S_ROT_NONE, H3S_ROT_REGULAR or H3S_ROT_SYLVESTER) in the low
// four bits, and above them a group size fixed at compile time (0: the group size of the call). A fixed group turns
// the butterfly's stage tests into constants, so the stages run as one straight block with no register copies at
// the joins of skipped stages.
constexpr int rot_kind(int rot) { return rot & 15; }
constexpr int rot_fixed(int rot) { return rot >> 4; }
constexpr int rot_with(int kind, int group) { return kind | (group << 4); }

struct QuantArgs {
    const void* x;
    int64_t M, C;
    const float* w;          // NULL: 1
    float eps;
    const int32_t* rows;     // NULL: table row 0
    const void* scale;       // scale and shift: both or neither
    const void* shift;
    int tab_dt;
    int h_dt;
    int rot;                 // H3S_ROT_NONE, H3S_ROT_REGULAR or H3S_ROT_SYLVESTER
    int group;
    float cg;                // fl(1 / sqrt(group))
    int8_t* q;
    float* s;
};

// ROT: the rotation kind (group size at run time); F: the side inputs (ROW_W, ROW_TAB, ROW_TAB32 or ROW_DYN, as in
// rowcore.h), or ROW_RAW: no norm, x itself is quantized, or ROW_SWIGLU: no norm, silu(gate) * up is quantized. The
// exact masks round h to bfloat16 (the type of the reference's scratch h and act); ROW_DYN takes h's type at run
// time.
//
// A unit (one block for rows of 256 or 512 lanes, one wavefront for 64-lane rows) quantizes the rows
// [unit * rpu, (unit + 1) * rpu). A lane works on the same chunks of every row, so the weight and the table row are
// decoded into registers once (the table row again only when rows[] changes), and with tables the next row's x is
// in flight while this one is computed.
template <int XDT, int CPL, int ROT, int F>
__global__ __launch_bounds__(512) void quant_kernel(QuantArgs A, int lshift, int64_t rpu) {
    constexpr bool ROTATED = rot_kind(ROT) != H3S_ROT_NONE;
    constexpr int V = Vec<XDT>::V;
    constexpr bool DYN = F & ROW_DYN;
    constexpr bool TW = DYN || (F & ROW_TAB32);
    constexpr bool SWI = F & ROW_SWIGLU;
    constexpr bool NORM = !(F & (ROW_RAW | ROW_SWIGLU));
    // a launch without tables gives each unit one row (persistent_launch keeps units only for table rows), so only
    // a kernel with tables holds registers for the next row's x: the others run at more wavefronts a SIMD (86
    // registers instead of 113 for the swiglu quantizer of 8192 features)
    constexpr bool PF = (F & (ROW_TAB | ROW_DYN)) != 0;
    __shared__ float red[2][8];
    const bool has_w = DYN ? A.w != nullptr : (F & ROW_W) != 0;
    const bool has_tab = DYN ? A.scale != nullptr : (F & ROW_TAB) != 0;
    const int tab_dt = (!DYN && (F & ROW_TAB32)) ? H3S_F32 : A.tab_dt;
    const int h_dt = DYN ? A.h_dt : H3S_BF16;
    const int L = 1 << lshift, W = L >> 6, lane = (int) (threadIdx.x & 63);
    const int t = (int) (threadIdx.x & (L - 1));
    const int64_t unit = L >= 256 ? (int64_t) blockIdx.x : (int64_t) blockIdx.x * (256 >> lshift) + (threadIdx.x >> lshift);
    const int64_t C = A.C, nch = C / V, r0 = unit * rpu, r1 = r0 + rpu < A.M ? r0 + rpu : A.M;
    if (r0 >= A.M) return;               // a unit with no rows (a whole block, or a 64-lane wavefront, which has no barrier)
    int64_t cc[CPL];
    bool ok[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = t + (int64_t) L * j;
        ok[j] = c < nch;
        cc[j] = ok[j] ? c : nch - 1;
    }
    // a row of x, and with SWIGLU the up half beside it (the gate half is xr)
    auto load_row = [&](uint4 (&xr)[CPL], uint4 (&ur)[CPL], int64_t row) {
        const uint4* xp = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(A.x) + row * C * (SWI ? 2 : 1) * (16 / V));
#pragma unroll
        for (int j = 0; j < CPL; ++j) xr[j] = ld_nt(xp + cc[j]);
        if constexpr (SWI)
#pragma unroll
            for (int j = 0; j < CPL; ++j) ur[j] = ld_nt(xp + nch + cc[j]);
    };
    // rounds a chunk to h's type (the reference's 16-bit scratch between its kernels)
    auto round_h = [&](float (&o)[V]) {
        if (h_dt == H3S_BF16) {
#pragma unroll
            for (int e = 0; e < V; e += 2) {
                const uint32_t p = pack_bf16(o[e], o[e + 1]);
                o[e] = bf16_lo(p);
                o[e + 1] = bf16_hi(p);
            }
        } else if (h_dt == H3S_F16) {
#pragma unroll
            for (int e = 0; e < V; e += 2) {
                const uint32_t p = pack_f16(o[e], o[e + 1]);
                o[e] = f16_lo(p);
                o[e + 1] = f16_hi(p);
            }
        }
    };
    // this row's and the next row's x (x0, x1; u0, u1 the up halves) and table row indices
    uint4 x0[CPL], u0[CPL];
    load_row(x0, u0, r0);
    int64_t t0 = has_tab && A.rows ? A.rows[r0] : 0;

    // ---- the weight and the table row, as floats: w, 1 + scale, shift ----
    float wv[CPL][V], s1[CPL][V], sh[CPL][V];
    if (has_w) {
        Raw<V, true> wr[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) fetch(wr[j], A.w, H3S_F32, cc[j] * V);
#pragma unroll
        for (int j = 0; j < CPL; ++j) decode(wr[j], H3S_F32, wv[j]);
    }
    int64_t tcur = -1;
    auto load_tables = [&](int64_t trow) {
        Raw<V, TW> sr[CPL], hr[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            fetch(sr[j], A.scale, tab_dt, trow * C + cc[j] * V);
            fetch(hr[j], A.shift, tab_dt, trow * C + cc[j] * V);
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            decode(sr[j], tab_dt, s1[j]);
            decode(hr[j], tab_dt, sh[j]);
#pragma unroll
            for (int e = 0; e < V; ++e) s1[j][e] = 1.0f + s1[j][e];
        }
    };

    // the normalization of a rotated group, with the sign the Sylvester cross-lane stages leave on this lane
    const int G = rot_fixed(ROT) ? rot_fixed(ROT) : A.group;
    const float cgs = rot_kind(ROT) == H3S_ROT_SYLVESTER ? A.cg * syl_sign<V>(lane, G) : A.cg;
    int slot = 0;   // consecutive reductions use alternate LDS slots
    for (int64_t row = r0; row < r1; ++row) {
        // the next row's x and table row index, in flight during this row
        uint4 x1[CPL], u1[CPL];
        int64_t t1 = 0;
        if (PF && row + 1 < r1) {
            load_row(x1, u1, row + 1);
            if (has_tab && A.rows) t1 = A.rows[row + 1];
        }
        if (has_tab && t0 != tcur) {
            load_tables(t0);
            tcur = t0;
        }

        float v[CPL][V];
#pragma unroll
        for (int j = 0; j < CPL; ++j) Vec<XDT>::unpack(x0[j], v[j]);

        // ---- rms_norm_mod into h's type ----
        if constexpr (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (ok[j])
#pragma unroll
                    for (int e = 0; e < V; ++e) ss = __builtin_fmaf(v[j][e], v[j][e], ss);
            const float inv = inv_root(row_sum(ss, red[slot], W), (float) C, A.eps);
            slot ^= 1;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (has_w) {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * inv * wv[j][e];
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * inv;
                }
                if (has_tab) {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * s1[j][e] + sh[j][e];
                }
                round_h(v[j]);
            }
        }
        // ---- swiglu into h's type: silu(g) * u, as h3s_swiglu computes it ----
        if constexpr (SWI) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                float u[V];
                Vec<XDT>::unpack(u0[j], u);
#pragma unroll
                for (int e = 0; e < V; ++e) v[j][e] = act_silu(v[j][e]) * u[e];
                round_h(v[j]);
            }
        }

        // ---- the block rotation, then the row's absolute maximum ----
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if constexpr (ROTATED) {
                if constexpr (rot_kind(ROT) == H3S_ROT_SYLVESTER) sylvester<V>(v[j], lane, G);
                else regular<V>(v[j], G);
#pragma unroll
                for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * cgs;
            }
            if (ok[j])
#pragma unroll
                for (int e = 0; e < V; ++e) m = fmaxf(m, fabsf(v[j][e]));
        }
        m = row_max(m, red[slot], W);
        slot ^= 1;
        const float sc = fmaxf(m / 127.0f, 1e-30f), r = 1.0f / sc;
        if (t == 0) A.s[row] = sc;

        // ---- the codes, V bytes a chunk ----
        int8_t* qrow = A.q + row * C;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if (!ok[j]) continue;
            const float* o = v[j];
            const uint32_t b0 = bytes4(code_of(o[0], sc, r), code_of(o[1], sc, r), code_of(o[2], sc, r), code_of(o[3], sc, r));
            if constexpr (V == 8) {
                const uint32_t b1 = bytes4(code_of(o[4], sc, r), code_of(o[5], sc, r), code_of(o[6], sc, r), code_of(o[7], sc, r));
                st_nt(qrow + cc[j] * 8, make_uint2(b0, b1));
            } else {
                st_nt(qrow + cc[j] * 4, b0);
            }
        }
        if constexpr (PF) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                x0[j] = x1[j];
                if constexpr (SWI) u0[j] = u1[j];
            }
        } else if (row + 1 < r1) {
            load_row(x0, u0, row + 1);
        }
        t0 = t1;
    }
}

// ---- one wavefront a row, for rows of exactly 64 CPL 16-byte chunks of a 16-bit type (2048 or 4096 features) ----
// The same arithmetic as quant_kernel, laid out so that the row's scalar work is done once: quant_kernel spreads
// such a row over four wavefronts, each of which repeats the row's statistics (the butterflies, the LDS combine
// and its barrier, the divisions and the square root). Here lane t of the wavefront holds chunks t + 64 j
// (j < CPL), every one inside the row, and the row statistics keep the order of the 256-lane layout that the oracle restates: chunk slot j
// belongs to canonical wavefront j % 4 (chunk t + 64 j is canonical lane (t + 64 j) % 256), so a lane keeps four
// partial sums, each summed over the wavefront by the butterfly and then combined as (w0 + w2) + (w1 + w3).
//
// Rows are dealt out grid-stride by wavefront: wavefront w of block b takes rows g, g + U, g + 2U, ... with
// g = b NW + w and U = NW x the blocks, so the rows in flight across the device form one contiguous window (a
// contiguous run per wavefront streams measurably slower), and at step k the block's wavefronts hold the
// neighbouring rows b NW + k U + [0, NW). The next row's x is in registers while a row is computed.
//
// The side inputs every wavefront of the block shares live in LDS, laid out [j][half][lane][4 floats] so that a
// wavefront's 16-byte reads are consecutive: the weight, and one decoded table row (1 + scale and shift), the
// table row of the block's first row at the current step. A step whose rows all share that table row (every step
// but those a segment boundary of rows[] cuts) is one round. Otherwise the block takes one round per distinct table
// row of the step, in the order of its rows: between two barriers it re-decodes the cached row when the round's
// differs, and the wavefronts whose rows use it run them (every wavefront takes the same rounds and barriers).
template <int CPL> constexpr size_t quant_wave_side_bytes(int f) {
    return (size_t) ((f & ROW_W) ? 1 : 0) * CPL * 2048 + (size_t) ((f & ROW_TAB) ? 2 : 0) * CPL * 2048;
}
// wavefronts a block: 8 with tables (one LDS copy of the side values serves more rows), else 4
constexpr int quant_wave_nw(int f) { return (f & ROW_TAB) ? 8 : 4; }
// ONE: the grid has a wavefront for every row, so each takes one row (108 registers for config 4's kernel, four
// wavefronts a SIMD); else the grid strides over the rows, with nothing prefetched either: four wavefronts a SIMD
// hide the loads (the registers of a prefetched next row would leave room for three). With tables and no rotation
// the kernel is held to four wavefronts a SIMD (120 registers, no spills).
template <int XDT, int CPL, int ROT, int F, bool ONE>
__global__ __launch_bounds__(512)
__attribute__((amdgpu_waves_per_eu((F & ROW_TAB) && rot_kind(ROT) == H3S_ROT_NONE ? 4 : 1)))
void quant_wave_kernel(QuantArgs A) {
    static_assert(XDT != H3S_F32 && !(F & (ROW_DYN | ROW_SWIGLU)), "quant_wave_kernel: 16-bit x, exact side inputs");
    constexpr int V = 8;
    constexpr bool ROTATED = rot_kind(ROT) != H3S_ROT_NONE;
    constexpr bool NORM = !(F & ROW_RAW);
    constexpr bool HASW = F & ROW_W;
    constexpr bool TAB = F & ROW_TAB;
    constexpr int TDT = (F & ROW_TAB32) ? H3S_F32 : H3S_BF16;
    constexpr int WOFF = 0, SOFF = HASW ? CPL * 512 : 0, HOFF = SOFF + CPL * 512;     // float offsets in side
    extern __shared__ __align__(16) float side[];
    constexpr int NW = quant_wave_nw(F);
    const int lane = (int) (threadIdx.x & 63);
    const int wave = (int) wave_uniform(threadIdx.x >> 6);
    const int64_t C = 64 * CPL * V;                         // the launch checks A.C against this
    const int64_t b0 = (int64_t) blockIdx.x * NW, U = (int64_t) gridDim.x * NW, M = A.M;
    if (b0 >= M) return;                                    // the whole block
    // chunk slot j: chunk 64 j + pos, pos = the lane (swap3 of the lane for the Sylvester rotation, whose stage 4
    // chunks apart then pairs lanes 7 apart: one DPP operand instead of two)
    constexpr bool SW = rot_kind(ROT) == H3S_ROT_SYLVESTER;
    const int pos = SW ? swap3(lane) : lane;
    int cc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) cc[j] = pos + 64 * j;
    // the side values of chunk j: 8 floats at ((j * 2 + half) * 64 + lane) * 4 of an array
    auto side_at = [&](int off, int j, int h) { return side + off + ((j * 2 + h) * 64 + lane) * 4; };
    auto put8 = [&](int off, int j, const float* f) {
        *reinterpret_cast<float4*>(side_at(off, j, 0)) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4*>(side_at(off, j, 1)) = make_float4(f[4], f[5], f[6], f[7]);
    };
    auto get8 = [&](int off, int j, float* f) {
        const float4 a = *reinterpret_cast<const float4*>(side_at(off, j, 0));
        const float4 b = *reinterpret_cast<const float4*>(side_at(off, j, 1));
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    };
    // one table row's 1 + scale and shift for chunk j, decoded from memory
    auto table8 = [&](int64_t trow, int j, float* s1, float* sh) {
        Raw<V, TDT == H3S_F32> sr, hr;
        fetch(sr, A.scale, TDT, trow * C + (int64_t) cc[j] * V);
        fetch(hr, A.shift, TDT, trow * C + (int64_t) cc[j] * V);
        decode(sr, TDT, s1);
        decode(hr, TDT, sh);
#pragma unroll
        for (int e = 0; e < V; ++e) s1[e] = 1.0f + s1[e];
    };
    // the block's side values (the weight with W, the table row trow): wavefront w decodes chunk slots w, w + NW, ...
    auto fill = [&](int64_t trow, bool with_w) {
        for (int j = wave; j < CPL; j += NW) {
#pragma unroll
            for (int jj = 0; jj < CPL; ++jj) {
                if (jj != j) continue;                       // a constant slot index for the register arrays
                if constexpr (HASW) {
                    if (with_w) {
                        Raw<V, true> wr;
                        fetch(wr, A.w, H3S_F32, (int64_t) cc[jj] * V);
                        float f[V];
                        decode(wr, H3S_F32, f);
                        put8(WOFF, jj, f);
                    }
                }
                if constexpr (TAB) {
                    float s1[V], sh[V];
                    table8(trow, jj, s1, sh);
                    put8(SOFF, jj, s1);
                    put8(HOFF, jj, sh);
                }
            }
        }
    };
    int64_t tcache = TAB && A.rows ? A.rows[b0] : 0;
    if constexpr (HASW || TAB) {
        fill(tcache, true);
        lds_barrier();
    }

    const int G = rot_fixed(ROT) ? rot_fixed(ROT) : A.group;
    const float cgs = SW ? A.cg * syl_sign<V>(pos, G) : A.cg;
    // a row's x: a base the whole wavefront shares (the row is the wavefront's) and a 32-bit unsigned byte offset
    // a lane, so the loads and stores take the scalar-base form and hold no 64-bit address registers (the row
    // passes through readfirstlane, which keeps the compiler from turning each chunk's address into an induction
    // variable of its own across the grid-stride loop)
    auto load_row = [&](uint4 (&xr)[CPL], int64_t row) {
        const char* xp = reinterpret_cast<const char*>(A.x) + wave_uniform(row) * C * 2;
#pragma unroll
        for (int j = 0; j < CPL; ++j) xr[j] = ld_nt(xp + (uint32_t) (cc[j] * 16));
    };
    // The table rows of each step's group of NW rows (rows g + [0, NW), g = b0 + k U, one a wavefront), 64 steps
    // at a time, one step a lane, taken out with readlane: the group's first row's (gix), this wavefront's (tix),
    // and a bit of uni set when the whole group shares one table row. rows[] is read once per 64 steps.
    int tix = 0, gix = 0;
    uint64_t uni = ~0ull;
    int64_t kbase = -64;
    auto group_rows = [&](int64_t k) {
        if (k - kbase >= 64) {
            kbase = k;
            const int64_t g = b0 + U * (k + lane);
            gix = g < M ? A.rows[g] : 0;
            tix = gix;
            bool same = true;
#pragma unroll
            for (int r = 1; r < NW; ++r) {
                const int t = g + r < M ? A.rows[g + r] : gix;
                same = same && t == gix;
                if (r == wave) tix = t;
            }
            uni = __builtin_amdgcn_ballot_w64(same);
        }
    };
    // One row, with the table row cached in LDS.
    auto process = [&](int64_t row) {
        uint4 x[CPL];
        load_row(x, row);
        float v[CPL][V];
#pragma unroll
        for (int j = 0; j < CPL; ++j) Vec<XDT>::unpack(x[j], v[j]);

        // ---- rms_norm_mod into bfloat16 (the reference's scratch h) ----
        if constexpr (NORM) {
            float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int e = 0; e < V; ++e) ss[j % 4] = __builtin_fmaf(v[j][e], v[j][e], ss[j % 4]);
            float w4[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) w4[g] = wave_sum<64, SW>(ss[g]);
            const float inv = inv_root((w4[0] + w4[2]) + (w4[1] + w4[3]), (float) C, A.eps);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if constexpr (HASW) {
                    float w[V];
                    get8(WOFF, j, w);
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * inv * w[e];
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * inv;
                }
                if constexpr (TAB) {
                    float s1[V], sh[V];
                    get8(SOFF, j, s1);
                    get8(HOFF, j, sh);
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * s1[e] + sh[e];
                }
#pragma unroll
                for (int e = 0; e < V; e += 2) {
                    const uint32_t p = pack_bf16(v[j][e], v[j][e + 1]);
                    v[j][e] = bf16_lo(p);
                    v[j][e + 1] = bf16_hi(p);
                }
                // with tables, one chunk's LDS reads at a time: the registers stay within four wavefronts a SIMD
                if constexpr (TAB) __builtin_amdgcn_sched_barrier(0);
            }
        }

        // ---- the block rotation, then the row's absolute maximum ----
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if constexpr (ROTATED) {
                if constexpr (SW) sylvester<V, true>(v[j], pos, G);
                else regular<V>(v[j], G);
#pragma unroll
                for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * cgs;
            }
#pragma unroll
            for (int e = 0; e < V; ++e) m = fmaxf(m, fabsf(v[j][e]));
        }
        m = wave_max<64>(m);
        const float sc = fmaxf(m / 127.0f, 1e-30f), r = 1.0f / sc;
        if (lane == 0) A.s[row] = sc;

        // ---- the codes, 8 bytes a chunk ----
        int8_t* qrow = A.q + wave_uniform(row) * C;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float* o = v[j];
            const uint32_t lo = bytes4(code_of(o[0], sc, r), code_of(o[1], sc, r), code_of(o[2], sc, r), code_of(o[3], sc, r));
            const uint32_t hi = bytes4(code_of(o[4], sc, r), code_of(o[5], sc, r), code_of(o[6], sc, r), code_of(o[7], sc, r));
            st_nt(qrow + (uint32_t) (cc[j] * 8), make_uint2(lo, hi));
        }
    };
    int64_t row = b0 + wave;
    if constexpr (ONE) {
        if (row < M) process(row);
        return;
    }
    for (int64_t k = 0, g = b0; g < M; row += U, g += U, ++k) {
        if constexpr (TAB) {
            int64_t first = 0, own = 0;
            bool same = true;
            if (A.rows) {
                group_rows(k);
                const int i = (int) (k - kbase);
                first = __builtin_amdgcn_readlane(gix, i);
                own = __builtin_amdgcn_readlane(tix, i);
                same = (uni >> i) & 1;
            }
            // One round for each distinct table row of the group, in the order of the group's rows: the block
            // refills its cached table row between barriers when it changes, and the wavefronts whose rows use it
            // run them. A group that shares one table row (every group but those a segment boundary cuts) is one
            // round; the others read their table rows again, as scalar loads. Every wavefront of the block takes
            // the same rounds and barriers.
            for (int r = 0; r < NW; ++r) {
                int64_t t = first;
                if (r > 0) {
                    if (same || g + r >= M) break;
                    t = A.rows[g + r];
                    bool seen = false;
                    for (int q = 0; q < r; ++q) seen = seen || A.rows[g + q] == t;
                    if (seen) continue;
                }
                if (t != tcache) {
                    lds_barrier();                           // every wavefront is done with the cached row
                    fill(t, false);
                    lds_barrier();
                    tcache = t;
                }
                if (row < M && own == t) process(row);
            }
        } else {
            if (row < M) process(row);
        }
    }
}

// The side-input masks compiled exactly for 16-bit inputs: none (h3s_int8_linear's quantizer), the weight
// (configs 1 and 4), the weight with 16-bit or float32 tables (config 5's front pass, the DiT's AdaLN). Every other
// call shape runs the ROW_DYN instantiation.
constexpr int kQuantNone = 0, kQuantW = ROW_W, kQuantWTab = ROW_W | ROW_TAB, kQuantWTab32 = ROW_W | ROW_TAB | ROW_TAB32,
              kQuantRaw = ROW_RAW, kQuantSwiglu = ROW_SWIGLU;

// The launch of quant_wave_kernel: blocks of 4 wavefronts (8 with tables, so one LDS copy of the side values
// serves more rows).
template <int XDT, int CPL, int ROT, int F> int quant_wave_one(Ctx* c, const char* fn, const QuantArgs& A) {
    const int threads = 64 * quant_wave_nw(F);
    const size_t lds = quant_wave_side_bytes<CPL>(F);
    const int64_t rows_blocks = (A.M + threads / 64 - 1) / (threads / 64);
    // One row a wavefront, nothing prefetched (config 4 at 47104 rows: 106 us, against 119 us grid-strided with the
    // next row in flight): without tables, and with tables whose one row serves every token (rows NULL), each block
    // decoding its side values once. With a table row per token, as many blocks as the device holds, grid-strided,
    // each refilling its cached table row when the rows' table row changes.
    if constexpr (F & ROW_TAB) {
        if (A.rows) {
            const void* k = (const void*) quant_wave_kernel<XDT, CPL, ROT, F, false>;
            const int64_t blocks = std::min<int64_t>((int64_t) c->cus * blocks_per_cu(k, threads, lds), rows_blocks);
            quant_wave_kernel<XDT, CPL, ROT, F, false><<<(unsigned) blocks, threads, lds, c->stream>>>(A);
            return launched(fn);
        }
    }
    quant_wave_kernel<XDT, CPL, ROT, F, true><<<(unsigned) rows_blocks, threads, lds, c->stream>>>(A);
    return launched(fn);
}
template <int XDT, int CPL> int quant_wave_launch(Ctx* c, const char* fn, const QuantArgs& A, int f) {
#define H3_QW(RR)                                                                          \
    if (f == kQuantNone) return quant_wave_one<XDT, CPL, RR, kQuantNone>(c, fn, A);         \
    if (f == kQuantW) return quant_wave_one<XDT, CPL, RR, kQuantW>(c, fn, A);               \
    if (f == kQuantWTab) return quant_wave_one<XDT, CPL, RR, kQuantWTab>(c, fn, A);         \
    if (f == kQuantWTab32) return quant_wave_one<XDT, CPL, RR, kQuantWTab32>(c, fn, A);     \
    return quant_wave_one<XDT, CPL, RR, kQuantRaw>(c, fn, A);
    if (A.rot == H3S_ROT_SYLVESTER && A.group == 128) { H3_QW(rot_with(H3S_ROT_SYLVESTER, 128)) }
    if (A.rot == H3S_ROT_SYLVESTER) { H3_QW(H3S_ROT_SYLVESTER) }
    if (A.rot == H3S_ROT_REGULAR) { H3_QW(H3S_ROT_REGULAR) }
    H3_QW(H3S_ROT_NONE)
#undef H3_QW
}

// what the quantizer runs on: rms_norm_mod of x, x itself, or swiglu of x
enum QuantMode { QUANT_NORM, QUANT_RAW, QUANT_SWIGLU };

// Launches the kernel for one input type; the plan comes from row_plan.
template <int XDT> int quant_launch(Ctx* c, const char* fn, const QuantArgs& A, int mode, RowPlan p) {
    int f = (A.w ? ROW_W : 0) | (A.scale ? ROW_TAB | (A.tab_dt == H3S_F32 ? ROW_TAB32 : 0) : 0);
    if (XDT == H3S_F32 || A.h_dt != H3S_BF16 || !(f == kQuantNone || f == kQuantW || f == kQuantWTab || f == kQuantWTab32))
        f = ROW_DYN;
    if (mode == QUANT_RAW) f = kQuantRaw;
    if (mode == QUANT_SWIGLU) f = XDT == H3S_F32 || A.h_dt != H3S_BF16 ? (ROW_SWIGLU | ROW_DYN) : kQuantSwiglu;
#define H3_QUANT_F(CC, RR, FF)                                                                      \
    {                                                                                                \
        const PersistentLaunch R = persistent_launch(c, (const void*) quant_kernel<XDT, CC, RR, FF>, A.M, p, A.scale != nullptr); \
        quant_kernel<XDT, CC, RR, FF><<<R.grid, R.threads, 0, c->stream>>>(A, R.lshift, R.rpu);    \
    }
#define H3_QUANT_R(CC, RR)                                                                           \
    if (f == kQuantRaw) { H3_QUANT_F(CC, RR, kQuantRaw); return launched(fn); }                     \
    if (f == kQuantSwiglu && A.rot == H3S_ROT_REGULAR && A.group == 256) {                           \
        H3_QUANT_F(CC, rot_with(H3S_ROT_REGULAR, 256), kQuantSwiglu);                                \
        return launched(fn);                                                                         \
    }                                                                                                \
    if (f == kQuantSwiglu) { H3_QUANT_F(CC, RR, kQuantSwiglu); return launched(fn); }               \
    if (f == (ROW_SWIGLU | ROW_DYN)) { H3_QUANT_F(CC, RR, ROW_SWIGLU | ROW_DYN); return launched(fn); } \
    if constexpr (XDT != H3S_F32) {                                                                  \
        if (f == kQuantNone) { H3_QUANT_F(CC, RR, kQuantNone); return launched(fn); }               \
        if (f == kQuantW) { H3_QUANT_F(CC, RR, kQuantW); return launched(fn); }                     \
        if (f == kQuantWTab) { H3_QUANT_F(CC, RR, kQuantWTab); return launched(fn); }               \
        if (f == kQuantWTab32) { H3_QUANT_F(CC, RR, kQuantWTab32); return launched(fn); }           \
    }                                                                                                \
    H3_QUANT_F(CC, RR, ROW_DYN);                                                                     \
    return launched(fn);
    // rows of 2048 or 4096 features of a 16-bit type with the exact side inputs, and enough of them (the context's
    // quant_wave_min, 8192) to give every wavefront several rows: one wavefront a row (fewer rows: four wavefronts
    // share each, which shortens a short launch)
    if constexpr (XDT != H3S_F32) {
        if ((f == kQuantNone || f == kQuantW || f == kQuantWTab || f == kQuantWTab32 || f == kQuantRaw) &&
            (A.C == 2048 || A.C == 4096) && A.M >= c->quant_wave_min) {
            if (A.C == 2048) return quant_wave_launch<XDT, 4>(c, fn, A, f);
            return quant_wave_launch<XDT, 8>(c, fn, A, f);
        }
    }
#define H3_QUANT_CPL(CC)                                                      \
    if (p.cpl == CC) {                                                        \
        if (A.rot == H3S_ROT_SYLVESTER) { H3_QUANT_R(CC, H3S_ROT_SYLVESTER) }  \
        else if (A.rot == H3S_ROT_REGULAR) { H3_QUANT_R(CC, H3S_ROT_REGULAR) } \
        else { H3_QUANT_R(CC, H3S_ROT_NONE) }                                 \
    }
    H3_QUANT_CPL(1)
    H3_QUANT_CPL(2)
    H3_QUANT_CPL(3)
    H3_QUANT_CPL(4)
#undef H3_QUANT_CPL
#undef H3_QUANT_R
#undef H3_QUANT_F
    return fail(std::string(fn) + ": no kernel for this row length");
}

}  // namespace h3
