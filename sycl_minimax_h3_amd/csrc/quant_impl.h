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
// the digit of stride 1, inside a chunk. Every digit forms t - 2 x as one fma, the oracle's (2 x is exact below
// 2^127, so it is the value of t - 2.0f * x)
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
        v[r] = __builtin_fmaf(-2.0f, quad<0xB1>(hi), t);
        v[r + 4] = __builtin_fmaf(-2.0f, quad<0xB1>(lo), t);
    }
}
// the digit of stride 4 with V = 4: x0..x3 in the four lanes of a quad, taken in order (quad_perm [a,a,a,a]); the
// mirror from the reversed quad ([3,2,1,0])
__device__ __forceinline__ void reg_quad(float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float t = ((quad<0x00>(v[e]) + quad<0x55>(v[e])) + quad<0xAA>(v[e])) + quad<0xFF>(v[e]);
        v[e] = __builtin_fmaf(-2.0f, quad<0x1B>(v[e]), t);
    }
}
// the digit whose four values sit in lanes S apart (a = (lane / S) % 4): the own pair x_a + x_(a^1), the other pair
// from the lanes 2S away, and the mirror x_(3-a) from the lane 3S away
template <int V, int S> __device__ __forceinline__ void reg_x(float (&v)[V]) {
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const float pv = v[e] + lane_xor<S>(v[e]);
        const float t = pv + lane_xor<2 * S>(pv);
        v[e] = __builtin_fmaf(-2.0f, lane_xor<3 * S>(v[e]), t);
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

// ---- the regular rotation of a group of 256 with a lane's 16 consecutive features in registers: the reference's
// work-item (kernels/h3sycl.cpp:408-456). The group's 16 lanes of a 16-lane DPP row hold its 16 runs of 16 features,
// run P = swap3(lane) & 15 in lane `lane` (a = features 0-7, b = 8-15). The digits of stride 1 and 4 are inside
// the lane, summed left to right; the digit of stride 16 pairs runs P ^ 1, P ^ 2, P ^ 3 = lanes ^ 1, ^ 2, ^ 3 (quad
// permutes); the digit of stride 64 runs P ^ 4, P ^ 8, P ^ 12 = lanes ^ 7, ^ 8, ^ 15 (swap3 turns position bit 2
// into lane xor 7: the half-row mirror, the row rotate by 8 and the row mirror), summed pairwise. Every partner
// value comes through the DPP operand of the add or fma that uses it: three instructions a value a digit, no LDS.
// pv = x + x[C1]; t = pv + pv[C2]; x = t - 2 x[C3] (one fma) for 8 values; s_nop 1: the two wait states a DPP read
// needs after the VALU write of its register
#define H3_DPP_ADD8(OUT, IN, CTRL)                                                                            \
    asm volatile("s_nop 1\n"                                                                                  \
                 "v_add_f32_dpp %0, %8, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                             \
                 "v_add_f32_dpp %1, %9, %9 " CTRL " row_mask:0xf bank_mask:0xf\n"                             \
                 "v_add_f32_dpp %2, %10, %10 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_add_f32_dpp %3, %11, %11 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_add_f32_dpp %4, %12, %12 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_add_f32_dpp %5, %13, %13 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_add_f32_dpp %6, %14, %14 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_add_f32_dpp %7, %15, %15 " CTRL " row_mask:0xf bank_mask:0xf"                              \
                 : "=&v"(OUT[0]), "=&v"(OUT[1]), "=&v"(OUT[2]), "=&v"(OUT[3]), "=&v"(OUT[4]), "=&v"(OUT[5]),     \
                   "=&v"(OUT[6]), "=&v"(OUT[7])                                                               \
                 : "v"(IN[0]), "v"(IN[1]), "v"(IN[2]), "v"(IN[3]), "v"(IN[4]), "v"(IN[5]), "v"(IN[6]), "v"(IN[7]))
#define H3_DPP_FMAC8(ACC, IN, M2, CTRL)                                                                        \
    asm volatile("s_nop 1\n"                                                                                  \
                 "v_fmac_f32_dpp %0, %8, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_fmac_f32_dpp %1, %9, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                           \
                 "v_fmac_f32_dpp %2, %10, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                          \
                 "v_fmac_f32_dpp %3, %11, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                          \
                 "v_fmac_f32_dpp %4, %12, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                          \
                 "v_fmac_f32_dpp %5, %13, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                          \
                 "v_fmac_f32_dpp %6, %14, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                          \
                 "v_fmac_f32_dpp %7, %15, %16 " CTRL " row_mask:0xf bank_mask:0xf"                             \
                 : "+v"(ACC[0]), "+v"(ACC[1]), "+v"(ACC[2]), "+v"(ACC[3]), "+v"(ACC[4]), "+v"(ACC[5]),         \
                   "+v"(ACC[6]), "+v"(ACC[7])                                                                 \
                 : "v"(IN[0]), "v"(IN[1]), "v"(IN[2]), "v"(IN[3]), "v"(IN[4]), "v"(IN[5]), "v"(IN[6]), "v"(IN[7]), \
                   "v"(M2))
// one cross-lane digit on 8 values x (in place)
#define H3_DIGIT8(X, C1, C2, C3)                                                                               \
    {                                                                                                          \
        float pv_[8], t_[8];                                                                                   \
        H3_DPP_ADD8(pv_, X, C1);                                                                               \
        H3_DPP_ADD8(t_, pv_, C2);                                                                              \
        H3_DPP_FMAC8(t_, X, m2, C3);                                                                           \
        _Pragma("unroll") for (int e_ = 0; e_ < 8; ++e_) X[e_] = t_[e_];                                       \
    }
__device__ __forceinline__ void regular256_pair(float (&a)[8], float (&b)[8]) {
    // stride 1: inside each chunk's two quads
    reg_in<8>(a);
    reg_in<8>(b);
    // stride 4: a[i], a[i + 4], b[i], b[i + 4]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = a[i], x1 = a[i + 4], x2 = b[i], x3 = b[i + 4];
        const float t = ((x0 + x1) + x2) + x3;
        a[i] = __builtin_fmaf(-2.0f, x3, t); a[i + 4] = __builtin_fmaf(-2.0f, x2, t);
        b[i] = __builtin_fmaf(-2.0f, x1, t); b[i + 4] = __builtin_fmaf(-2.0f, x0, t);
    }
    const float m2 = -2.0f;
    // stride 16: lanes ^ 1, ^ 2, ^ 3
    H3_DIGIT8(a, "quad_perm:[1,0,3,2]", "quad_perm:[2,3,0,1]", "quad_perm:[3,2,1,0]")
    H3_DIGIT8(b, "quad_perm:[1,0,3,2]", "quad_perm:[2,3,0,1]", "quad_perm:[3,2,1,0]")
    // stride 64: lanes ^ 7, ^ 8, ^ 15
    H3_DIGIT8(a, "row_half_mirror", "row_ror:8", "row_mirror")
    H3_DIGIT8(b, "row_half_mirror", "row_ror:8", "row_mirror")
}
#undef H3_DIGIT8
#undef H3_DPP_FMAC8
#undef H3_DPP_ADD8

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
    void* h = nullptr;       // ROW_OUTH: the bfloat16 rows h [M, C] (then q and s are unused)
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
        const float sc = fmaxf(div127(m), 1e-30f), r = 1.0f / sc;
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

// ---- one or more wavefronts a row, for rows of a 16-bit type whose chunk count the kernel fixes ----
// The same arithmetic as quant_kernel, laid out so that the row's scalar work is done once: quant_kernel spreads
// a row of 256 or more chunks over four or eight wavefronts, each of which repeats the row's statistics (the
// butterflies, the LDS combine and its barrier, the divisions and the square root). Here lane t of wavefront s of
// the row's WPR holds chunks t + 64 (WPR j + s) (j < CPL); in the row's last slots only the lanes whose chunk is
// below the row's NCH chunks hold one (5376 features, one wavefront a row: 10 whole slots and half of an eleventh),
// the others load a copy of the row's last chunk and never use it. A rotation group is whole inside the valid lanes
// (a group size divides C and 64 V), so it never mixes a copy with a chunk.
//
// Norm: the row statistics keep the order of the 256-lane layout that the oracle restates: chunk slot j belongs to
// canonical wavefront j % 4 (chunk t + 64 j is canonical lane (t + 64 j) % 256), so a lane keeps four partial sums,
// each summed over the wavefront by the butterfly and then combined as (w0 + w2) + (w1 + w3); with two wavefronts a
// row each forms its own two (w0 + w2, w1 + w3) and they meet in LDS. With ROW_OUTH the kernel is h3s_rms_norm_mod:
// it stores the bfloat16 row h itself and computes no codes.
//
// Several wavefronts a row: each wavefront's maximum goes to LDS, and after one barrier every wavefront of the row
// takes the maximum of the row's. The block's side values (below) hold the table row of its first row; a row of
// another table row reads its table values from memory.
//
// Rows are dealt out by wavefront (group): group w of block b takes row g = b R + w (R rows a block step) with ONE,
// else rows g, g + U, g + 2U, ... (U = R x the blocks: the rows in flight across the device form one contiguous
// window; a contiguous run per wavefront streams measurably slower).
//
// The side inputs every wavefront of the block shares live in LDS, laid out [j][half][lane][4 floats] so that a
// wavefront's 16-byte reads are consecutive: the weight, and one decoded table row (1 + scale and shift), the
// table row of the block's first row at the current step. A step whose rows all share that table row (every step
// but those a segment boundary of rows[] cuts) is one round. Otherwise the block takes one round per distinct table
// row of the step, in the order of its rows: between two barriers it re-decodes the cached row when the round's
// differs, and the wavefronts whose rows use it run them (every wavefront takes the same rounds and barriers).
template <int CPL, int WPR = 1> constexpr size_t quant_wave_side_bytes(int f) {
    return ((size_t) ((f & ROW_W) ? 1 : 0) + (size_t) ((f & ROW_TAB) ? 2 : 0)) * WPR * CPL * 2048;
}
// wavefronts a block: 8 with tables (one LDS copy of the side values serves more rows) or two or four a row, a row's
// own with more, else 4
enum : int { QW_ROUNDS = 0, QW_ONE = 1, QW_STREAM = 2 };
constexpr int quant_wave_nw(int f, int wpr, int mode) {
    // several wavefronts a row with no side values to share: a block is one row, so the blocks resident on a CU follow
    // the registers (the 5376-feature quantizer, two wavefronts a row: 54.7 against 57.4 us at 16896 rows in blocks of
    // four rows)
    if (!(f & (ROW_W | ROW_TAB)) && wpr > 1 && mode == QW_ONE) return wpr;
    return wpr > 4 || wpr == 3 ? wpr * (8 / wpr > 0 ? 8 / wpr : 1) : (f & ROW_TAB) || wpr > 1 ? 8 : 4;
}
// How a launch deals out its rows:
//   QW_ONE     the grid has a wavefront (group) for every row, so each takes one row (108 registers for config 4's
//              kernel, four wavefronts a SIMD);
//   QW_ROUNDS  one wavefront a row, the grid strided over the rows with nothing prefetched (four wavefronts a SIMD
//              hide the loads), a table row per token cached in LDS and refilled in rounds (below). With tables and no
//              rotation (and at most 8 slots) the kernel is held to four wavefronts a SIMD (120 registers, no spills);
//   QW_STREAM  as many blocks as the device holds, grid-strided, each group of wavefronts taking rows g, g + U, ...
//              with nothing prefetched; the block's side values (the weight, one table row) are decoded into LDS once
//              and refilled only when the table row of a step's first row changes (the norm at the hidden width: each
//              block of four rows had decoded 63 KiB of float32 weight and tables).
// The body of quant_wave_kernel for the blocks [blk0, ...) of one layout: block blk takes rows row0 + blk R ... (R rows
// a block step); NW wavefronts a block.
template <int XDT, int CPL, int ROT, int F, int MODE, int NCH, int WPR, bool PAIR, int NW>
__device__ __forceinline__ void quant_wave_body(const QuantArgs& A, int64_t blk, int64_t row0) {
    constexpr bool ONE = MODE == QW_ONE;
    static_assert(XDT != H3S_F32 && !(F & ROW_DYN), "quant_wave_kernel: 16-bit x, exact side inputs");
    static_assert(PAIR ? NCH > 128 * WPR * (CPL / 2 - 1) && NCH <= 128 * WPR * (CPL / 2)
                       : NCH > 64 * WPR * (CPL - 1) && NCH <= 64 * WPR * CPL, "quant_wave_kernel: NCH reaches the last slots");
    static_assert(WPR == 1 || (MODE != QW_ROUNDS && ((F & (ROW_RAW | ROW_SWIGLU)) || WPR == 2 || (WPR == 4 && !PAIR))),
                  "quant_wave_kernel: several wavefronts a row: the quantizer on x or swiglu(x), or the norm, two a row "
                  "(four a row one chunk a lane)");
    static_assert(NW % WPR == 0, "quant_wave_kernel: whole rows a block");
    static_assert(!PAIR || (ROT == rot_with(H3S_ROT_REGULAR, 256) && CPL % 2 == 0), "quant_wave_kernel: pairs for regular 256");
    constexpr int V = 8;
    constexpr bool ROTATED = rot_kind(ROT) != H3S_ROT_NONE;
    constexpr bool SWI = F & ROW_SWIGLU;
    constexpr bool NORM = !(F & (ROW_RAW | ROW_SWIGLU));
    constexpr bool OUTH = NORM && (F & ROW_OUTH);
    constexpr bool HASW = F & ROW_W;
    constexpr bool TAB = F & ROW_TAB;
    constexpr int TDT = (F & ROW_TAB32) ? H3S_F32 : H3S_BF16;
    constexpr int WOFF = 0, SOFF = HASW ? WPR * CPL * 512 : 0, HOFF = SOFF + WPR * CPL * 512;   // float offsets in side
    constexpr int RPB = NW / WPR;
    // NCH chunks a row; PAIR: slot pair p of wavefront s holds run pair k = WPR p + s (chunks 128 k + [0, 128))
    static_assert(!NORM || (NCH >= 256 && NCH <= 1024), "quant_wave_kernel: the norm's canonical order of 256 lanes");
    extern __shared__ __align__(16) float side[];
    __shared__ float wmax[NW];
    __shared__ float wsum[NW][2];
    const int lane = (int) (threadIdx.x & 63);
    const int wave = (int) wave_uniform(threadIdx.x >> 6);
    const int ws = wave % WPR, wr = wave / WPR;             // this wavefront's share of its row, and the row's group
    const int64_t C = (int64_t) NCH * V;                     // the launch checks A.C against this
    const int64_t b0 = row0 + blk * RPB, U = (int64_t) gridDim.x * RPB, M = A.M;   // (U: grid-strided, row0 0)
    if (b0 >= M) return;                                    // the whole block
    // chunk slot j: chunk 64 (WPR j + ws) + pos, pos = the lane (swap3 of the lane for the Sylvester rotation, whose
    // stage 4 chunks apart then pairs lanes 7 apart: one DPP operand instead of two; and for pairs, whose digit of
    // stride 64 features then pairs lanes 7, 8 and 15 apart)
    constexpr bool SW = rot_kind(ROT) == H3S_ROT_SYLVESTER || PAIR;
    const int pos = SW ? swap3(lane) : lane;
    // slot j of the row's wavefront s: its chunk, and whether it is inside the row (the row's last slots may be
    // partial or empty); chunk_of gives the row's last chunk for a lane past the row
    auto raw_chunk = [&](int s_, int j) {
        return PAIR ? 128 * (WPR * (j / 2) + s_) + 2 * pos + (j & 1) : pos + 64 * (WPR * j + s_);
    };
    auto valid_of = [&](int s_, int j) {
        // whole slots are decided at compile time; only the row's last ones test the lane
        if (PAIR ? 128 * (WPR * (j / 2) + WPR) <= NCH : 64 * (WPR * j + WPR) <= NCH) return true;
        return raw_chunk(s_, j) < NCH;
    };
    auto chunk_of = [&](int s_, int j) { return valid_of(s_, j) ? raw_chunk(s_, j) : NCH - 1; };
    auto valid = [&](int j) { return valid_of(ws, j); };
    int cc[CPL];                                            // the chunks this wavefront loads
#pragma unroll
    for (int j = 0; j < CPL; ++j) cc[j] = chunk_of(ws, j);
    // the side values of slot j of the row's wavefront s: 8 floats at (((s CPL + j) * 2 + half) * 64 + lane) * 4 of an
    // array (each of the row's wavefronts has its own slots)
    auto side_at = [&](int off, int sj, int h) { return side + off + ((sj * 2 + h) * 64 + lane) * 4; };
    auto put8 = [&](int off, int sj, const float* f) {
        *reinterpret_cast<float4*>(side_at(off, sj, 0)) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4*>(side_at(off, sj, 1)) = make_float4(f[4], f[5], f[6], f[7]);
    };
    auto get8 = [&](int off, int j, float* f) {
        const float4 a = *reinterpret_cast<const float4*>(side_at(off, ws * CPL + j, 0));
        const float4 b = *reinterpret_cast<const float4*>(side_at(off, ws * CPL + j, 1));
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    };
    // one table row's 1 + scale and shift for chunk c, decoded from memory
    auto table8 = [&](int64_t trow, int c, float* s1, float* sh) {
        Raw<V, TDT == H3S_F32> sr, hr;
        fetch(sr, A.scale, TDT, trow * C + (int64_t) c * V);
        fetch(hr, A.shift, TDT, trow * C + (int64_t) c * V);
        decode(sr, TDT, s1);
        decode(hr, TDT, sh);
#pragma unroll
        for (int e = 0; e < V; ++e) s1[e] = 1.0f + s1[e];
    };
    // the block's side values (the weight with W, the table row trow): wavefront w decodes slots w, w + NW, ... of
    // the row's WPR CPL slots
    auto fill = [&](int64_t trow, bool with_w) {
        for (int sj = wave; sj < WPR * CPL; sj += NW) {
            const int c = chunk_of(sj / CPL, sj % CPL);
            if constexpr (HASW) {
                if (with_w) {
                    Raw<V, true> wr;
                    fetch(wr, A.w, H3S_F32, (int64_t) c * V);
                    float f[V];
                    decode(wr, H3S_F32, f);
                    put8(WOFF, sj, f);
                }
            }
            if constexpr (TAB) {
                float s1[V], sh[V];
                table8(trow, c, s1, sh);
                put8(SOFF, sj, s1);
                put8(HOFF, sj, sh);
            }
        }
    };
    const int G = rot_fixed(ROT) ? rot_fixed(ROT) : A.group;
    const float cgs = rot_kind(ROT) == H3S_ROT_SYLVESTER ? A.cg * syl_sign<V>(pos, G) : A.cg;
    // a row's x: a base the whole wavefront shares (the row is the wavefront's) and a 32-bit unsigned byte offset
    // a lane, so the loads and stores take the scalar-base form and hold no 64-bit address registers (the row
    // passes through readfirstlane, which keeps the compiler from turning each chunk's address into an induction
    // variable of its own across the grid-stride loop). With SWIGLU the row is [gate | up], 2 C features.
    auto load_row = [&](uint4 (&xr)[CPL], uint4 (&ur)[CPL], int64_t row) {
        const char* xp = reinterpret_cast<const char*>(A.x) + wave_uniform(row) * C * 2 * (SWI ? 2 : 1);
#pragma unroll
        for (int j = 0; j < CPL; ++j) xr[j] = ld_nt(xp + (uint32_t) (cc[j] * 16));
        if constexpr (SWI)
#pragma unroll
            for (int j = 0; j < CPL; ++j) ur[j] = ld_nt(xp + (uint32_t) ((NCH + cc[j]) * 16));
    };
    const int64_t M1 = M - 1;
    int64_t tcache = TAB && A.rows ? A.rows[b0] : 0;
    if constexpr (HASW || TAB) {
        fill(tcache, true);
        lds_barrier();
    }
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
    // One row (its share), with the table row cached in LDS; live false: a row past the end (ONE with several
    // wavefronts a row), computed on a copy for the barrier and not stored.
    // tab_lds: the row's table row is the one cached in LDS (else its values are read from memory, chunk by chunk)
    auto compute = [&](const uint4 (&x)[CPL], const uint4 (&u)[CPL], int64_t row, bool live, bool tab_lds) {
        float v[CPL][V];
#pragma unroll
        for (int j = 0; j < CPL; ++j) Vec<XDT>::unpack(x[j], v[j]);

        // ---- rms_norm_mod into bfloat16 (the reference's scratch h) ----
        if constexpr (NORM) {
            // PAIR: chunk 128 k + 2 pos + h is canonical lane 2 (pos % 32) + h of canonical wavefront 2 (k % 2) +
            // pos / 32, so a lane keeps a partial sum for each (k % 2, h); each is summed over its half wave (the
            // canonical offsets 32 .. 2 are the position offsets 16 .. 1), the two h then added (offset 1), and the
            // halves hold canonical wavefronts (0, 2) and (1, 3): (w0 + w2) + (w1 + w3) across them
            float ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (valid(j)) {
                    // (two wavefronts a row: a wavefront's run pairs all have k % 2 = its share s; one chunk a lane,
                    // slot j of wavefront s is canonical wavefront (2 j + s) % 4, its partial j % 2)
                    const int q = PAIR ? (WPR == 2 ? (j & 1) : ((j / 2) % 2) * 2 + (j & 1)) : WPR == 4 ? 0 : WPR == 2 ? j % 2 : j % 4;
#pragma unroll
                    for (int e = 0; e < V; ++e) ss[q] = __builtin_fmaf(v[j][e], v[j][e], ss[q]);
                }
            float tot;
            if constexpr (PAIR && WPR == 2) {
                // wavefront s holds the run pairs k = 2 p + s, so k % 2 = s: its halves hold canonical wavefronts 2 s
                // and 2 s + 1 (its partials ss[0], ss[1] by h); the row's two wavefronts meet in LDS for
                // (w0 + w2) + (w1 + w3)
                const float w = wave_sum<32, SW>(ss[0]) + wave_sum<32, SW>(ss[1]);
                if ((lane & 31) == 0) wsum[wave][lane >> 5] = w;
                lds_barrier();
                const int b = wr * 2;
                tot = (wsum[b][0] + wsum[b + 1][0]) + (wsum[b][1] + wsum[b + 1][1]);
            } else if constexpr (WPR == 4) {
                // wavefront s holds canonical wavefront s (its slots j are chunks 64 (4 j + s) + pos): they meet in
                // LDS for (w0 + w2) + (w1 + w3)
                const float w = wave_sum<64, SW>(ss[0]);
                if (lane == 0) wsum[wave][0] = w;
                lds_barrier();
                const int b = wr * 4;
                tot = (wsum[b][0] + wsum[b + 2][0]) + (wsum[b + 1][0] + wsum[b + 3][0]);
            } else if constexpr (WPR == 2) {
                // wavefront s holds canonical wavefronts s (ss[0]) and s + 2 (ss[1]): w0 + w2 in the first, w1 + w3
                // in the second, met in LDS
                const float w = wave_sum<64, SW>(ss[0]) + wave_sum<64, SW>(ss[1]);
                if (lane == 0) wsum[wave][0] = w;
                lds_barrier();
                tot = wsum[wr * 2][0] + wsum[wr * 2 + 1][0];
            } else if constexpr (PAIR) {
                float w4[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) w4[g] = wave_sum<32, SW>(ss[g]);
                const float half = (w4[0] + w4[1]) + (w4[2] + w4[3]);
                tot = half + xor_lane<32>(half);
            } else {
                float w4[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) w4[g] = wave_sum<64, SW>(ss[g]);
                tot = (w4[0] + w4[2]) + (w4[1] + w4[3]);
            }
            const float inv = inv_root(tot, (float) C, A.eps);
            uint16_t* hrow = OUTH ? reinterpret_cast<uint16_t*>(A.h) + wave_uniform(row) * C : nullptr;
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
                    // (one wavefront a row takes rows[] grid-strided, with every table row through LDS)
                    if (WPR == 1 || tab_lds) {
                        get8(SOFF, j, s1);
                        get8(HOFF, j, sh);
                    } else {
                        table8(A.rows[row], cc[j], s1, sh);
                    }
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * s1[e] + sh[e];
                }
                uint32_t p[V / 2];
#pragma unroll
                for (int e = 0; e < V; e += 2) {
                    p[e / 2] = pack_bf16(v[j][e], v[j][e + 1]);
                    v[j][e] = bf16_lo(p[e / 2]);
                    v[j][e + 1] = bf16_hi(p[e / 2]);
                }
                if constexpr (OUTH) {
                    if (live && valid(j)) st_nt(hrow + (uint32_t) (cc[j] * 8), make_uint4(p[0], p[1], p[2], p[3]));
                }
                // with tables, one chunk's LDS reads at a time: the registers stay within four wavefronts a SIMD
                if constexpr (TAB) __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (OUTH) return;
        }
        // ---- swiglu into bfloat16, as h3s_swiglu computes it (the MLP's scratch act) ----
        if constexpr (SWI) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                float uu[V];
                Vec<XDT>::unpack(u[j], uu);
#pragma unroll
                for (int e = 0; e < V; ++e) v[j][e] = act_silu(v[j][e]) * uu[e];
#pragma unroll
                for (int e = 0; e < V; e += 2) {
                    const uint32_t p = pack_bf16(v[j][e], v[j][e + 1]);
                    v[j][e] = bf16_lo(p);
                    v[j][e + 1] = bf16_hi(p);
                }
            }
        }

        // ---- the block rotation, then the row's absolute maximum ----
        // P2: the regular rotation of a fixed group of 256, whose fl(1 / sqrt(256)) = 2^-4 is a power of two. The
        // values are then left unscaled: y = v 2^-4 exactly, so y / s = v / (16 s) exactly, and code_of(v, 16 s,
        // fl(1 / s) / 16) forms every intermediate 16 times that of code_of(y, s, fl(1 / s)) - the same roundings,
        // the same bits - as long as no intermediate is subnormal. A row whose unscaled maximum is below 2^-60 (its
        // codes' residuals could be) takes the scaled values as written.
        constexpr bool P2 = rot_kind(ROT) == H3S_ROT_REGULAR && rot_fixed(ROT) == 256;
        float m = 0.0f;
        if constexpr (PAIR) {
#pragma unroll
            for (int j = 0; j < CPL; j += 2) regular256_pair(v[j], v[j + 1]);
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if constexpr (ROTATED) {
                if constexpr (!PAIR) {
                    if constexpr (SW) sylvester<V, true>(v[j], pos, G);
                    else regular<V>(v[j], G);
                }
                if constexpr (!P2)
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * cgs;
            }
            if (valid(j))
#pragma unroll
                for (int e = 0; e < V; ++e) m = fmaxf(m, fabsf(v[j][e]));
        }
        m = wave_max<64>(m);
        if constexpr (WPR > 1) {
            // the row's wavefronts meet once: every wavefront of the block reaches this barrier (ONE)
            if (lane == 0) wmax[wave] = m;
            lds_barrier();
#pragma unroll
            for (int s = 0; s < WPR; ++s) m = fmaxf(m, wmax[wr * WPR + s]);
        }
        bool unscaled = false;
        if constexpr (P2) {
            // the maximum of the scaled values, fl(max |v| 2^-4) (rounding is monotonic)
            unscaled = m >= 0x1p-60f;
            if (!unscaled) {
#pragma unroll
                for (int j = 0; j < CPL; ++j)
#pragma unroll
                    for (int e = 0; e < V; ++e) v[j][e] = v[j][e] * cgs;
            }
            m = m * cgs;
        }
        const float sc = fmaxf(div127(m), 1e-30f), r = 1.0f / sc;
        if (!live) return;
        if (lane == 0 && ws == 0) A.s[row] = sc;
        const float sq = unscaled ? sc * 16.0f : sc, rq = unscaled ? r * 0.0625f : r;   // the codes' divisor

        // ---- the codes, 8 bytes a chunk; a lane's run pair (two consecutive chunks) as one 16-byte store, so each
        // store instruction writes whole lines (two 8-byte halves 16 bytes apart wrote up to 17 % more bytes) ----
        int8_t* qrow = A.q + wave_uniform(row) * C;
        auto codes8 = [&](const float* o) {
            return make_uint2(bytes4(code_of(o[0], sq, rq), code_of(o[1], sq, rq), code_of(o[2], sq, rq), code_of(o[3], sq, rq)),
                              bytes4(code_of(o[4], sq, rq), code_of(o[5], sq, rq), code_of(o[6], sq, rq), code_of(o[7], sq, rq)));
        };
#pragma unroll
        for (int j = 0; j < CPL; j += PAIR ? 2 : 1) {
            if (!valid(j)) continue;                      // (a pair's two chunks are inside the row or past it together)
            const uint2 a = codes8(v[j]);
            if constexpr (PAIR) {
                const uint2 b = codes8(v[j + 1]);
                st_nt(qrow + (uint32_t) (cc[j] * 8), make_uint4(a.x, a.y, b.x, b.y));
            } else {
                st_nt(qrow + (uint32_t) (cc[j] * 8), a);
            }
        }
    };
    auto process = [&](int64_t row, bool live, bool tab_lds) {
        uint4 x[CPL], u[CPL];
        load_row(x, u, row);
        compute(x, u, row, live, tab_lds);
    };
    int64_t row = b0 + wr;
    if constexpr (MODE == QW_STREAM) {
        // Steps g = b0, b0 + U, ...: this group's row g + wr. Every wavefront of the block takes every step (a row past
        // the end is computed on a copy and not stored), so the row barriers and the refills below match. The block's
        // cached table row is that of the step's first row (a uniform value): a step whose first row has another one
        // refills the cache between two barriers; a row whose table row differs from the cached one (a segment
        // boundary of rows[] inside the step) reads its table values from memory.
        for (int64_t g = b0; g < M; g += U) {
            const int64_t rc = g + wr < M ? g + wr : M1;
            bool tab_lds = true;
            if constexpr (TAB) {
                if (A.rows) {
                    const int64_t tg = A.rows[g];
                    if (tg != tcache) {
                        lds_barrier();                    // every wavefront is done with the cached row
                        fill(tg, false);
                        lds_barrier();
                        tcache = tg;
                    }
                    tab_lds = A.rows[rc] == tcache;
                }
            }
            process(rc, g + wr < M, tab_lds);
        }
        return;
    }
    if constexpr (ONE) {
        // the block's side values hold the table row of its first row; a row of another table row (one a segment
        // boundary of rows[] puts in the block) reads its table values from memory
        const int64_t rc = row < M ? row : M - 1;
        const bool tab_lds = !TAB || !A.rows || A.rows[rc] == tcache;
        if constexpr (WPR > 1) process(rc, row < M, tab_lds);
        else if (row < M) process(row, true, tab_lds);
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
                if (row < M && own == t) process(row, true, true);
            }
        } else {
            if (row < M) process(row, true, true);
        }
    }
}

// TAIL > 1: the blocks from tail_blk0 on take the rows from tail_row0 on with TAIL wavefronts a row (CPL / TAIL
// slots each, the same chunks and the same arithmetic and order), so the launch's last rows, which run on a
// partly idle device, end sooner.
template <int XDT, int CPL, int ROT, int F, int MODE, int NCH, int WPR = 1, bool PAIR = false, int TAIL = 1>
__global__ __launch_bounds__(512)
__attribute__((amdgpu_waves_per_eu((F & ROW_TAB) && rot_kind(ROT) == H3S_ROT_NONE && CPL <= 8 && MODE == QW_ROUNDS ? 4 : 1)))
void quant_wave_kernel(QuantArgs A, int64_t tail_blk0, int64_t tail_row0) {
    constexpr int NW = quant_wave_nw(F, WPR, MODE);
    static_assert(NW * 64 <= 512, "quant_wave_kernel: a block within the launch bound");
    if constexpr (TAIL > 1) {
        static_assert(MODE == QW_ONE && WPR == 1 && !PAIR && CPL % TAIL == 0, "quant_wave_kernel: a tail of one-wavefront rows");
        if ((int64_t) blockIdx.x >= tail_blk0) {
            quant_wave_body<XDT, CPL / TAIL, ROT, F, QW_ONE, NCH, TAIL, PAIR, NW>(A, (int64_t) blockIdx.x - tail_blk0, tail_row0);
            return;
        }
    }
    quant_wave_body<XDT, CPL, ROT, F, MODE, NCH, WPR, PAIR, NW>(A, blockIdx.x, 0);
}

// The side-input masks compiled exactly for 16-bit inputs: none (h3s_int8_linear's quantizer), the weight
// (configs 1 and 4), the weight with 16-bit or float32 tables (config 5's front pass, the DiT's AdaLN). Every other
// call shape runs the ROW_DYN instantiation.
constexpr int kQuantNone = 0, kQuantW = ROW_W, kQuantWTab = ROW_W | ROW_TAB, kQuantWTab32 = ROW_W | ROW_TAB | ROW_TAB32,
              kQuantRaw = ROW_RAW, kQuantSwiglu = ROW_SWIGLU;

// The launch of quant_wave_kernel: blocks of 4 wavefronts (8 with tables, so one LDS copy of the side values
// serves more rows, or with several wavefronts a row).
template <int XDT, int CPL, int ROT, int F, int NCH, int WPR, bool PAIR = false, int TAIL = 1, int MODE = QW_ONE>
int quant_wave_one(Ctx* c, const char* fn, const QuantArgs& A) {
    constexpr int NW = quant_wave_nw(F, WPR, MODE), RPB = NW / WPR;
    const int threads = 64 * NW;
    const size_t lds = quant_wave_side_bytes<CPL, WPR>(F);
    const int64_t rows_blocks = (A.M + RPB - 1) / RPB;
    if constexpr (MODE == QW_STREAM) {
        const void* k = (const void*) quant_wave_kernel<XDT, CPL, ROT, F, MODE, NCH, WPR, PAIR>;
        const int64_t blocks = std::min<int64_t>((int64_t) c->cus * blocks_per_cu(k, threads, lds), rows_blocks);
        if (blocks < 1) return fail(std::string(fn) + ": the streamed row kernel fits no compute unit");
        quant_wave_kernel<XDT, CPL, ROT, F, MODE, NCH, WPR, PAIR><<<(unsigned) blocks, threads, lds, c->stream>>>(A, blocks, A.M);
        return launched(fn);
    } else {
    // One row a wavefront, nothing prefetched (config 4 at 47104 rows: 106 us, against 119 us grid-strided with the
    // next row in flight): without tables, and with tables whose one row serves every token (rows NULL), each block
    // decoding its side values once. With a table row per token, as many blocks as the device holds, grid-strided,
    // each refilling its cached table row when the rows' table row changes.
    if constexpr ((F & ROW_TAB) && WPR == 1) {
        if (A.rows) {
            const void* k = (const void*) quant_wave_kernel<XDT, CPL, ROT, F, QW_ROUNDS, NCH, WPR, PAIR>;
            const int64_t blocks = std::min<int64_t>((int64_t) c->cus * blocks_per_cu(k, threads, lds), rows_blocks);
            quant_wave_kernel<XDT, CPL, ROT, F, QW_ROUNDS, NCH, WPR, PAIR><<<(unsigned) blocks, threads, lds, c->stream>>>(A, blocks, A.M);
            return launched(fn);
        }
    }
    // With a tail form: the blocks that fill whole rounds of the device take one row a wavefront, and the rows of
    // a last round at most a quarter full TAIL wavefronts a row (config 4 at 16896 rows, 0.125 of a round: 43.4
    // against 44.3 us, config 5a 41.2 against 42.1; at 47104 rows, half a round, the tail form measured 4 % slower)
    int64_t main_blocks = rows_blocks, tail_blocks = 0;
    if constexpr (TAIL > 1) {
        const void* k = (const void*) quant_wave_kernel<XDT, CPL, ROT, F, QW_ONE, NCH, WPR, PAIR, TAIL>;
        const int64_t round = (int64_t) c->cus * blocks_per_cu(k, threads, lds);
        const int64_t full = rows_blocks / round * round;
        if (full > 0 && full < rows_blocks && 4 * (rows_blocks - full) <= round) {
            main_blocks = full;
            tail_blocks = (A.M - full * RPB + (NW / TAIL) - 1) / (NW / TAIL);
        }
    }
    quant_wave_kernel<XDT, CPL, ROT, F, QW_ONE, NCH, WPR, PAIR, TAIL>
        <<<(unsigned) (main_blocks + tail_blocks), threads, lds, c->stream>>>(A, main_blocks, main_blocks * RPB);
    return launched(fn);
    }
}
// rows of 2048 or 4096 features (CPL 4 or 8, every slot whole): the norm with its side inputs, or the quantizer on x;
// at 4096 features the norm's launches end with the last partial round four wavefronts a row
template <int XDT, int CPL> int quant_wave_launch(Ctx* c, const char* fn, const QuantArgs& A, int f) {
    constexpr int TL = CPL == 8 ? 4 : 1;
#define H3_QW(RR)                                                                                  \
    if (f == kQuantNone) return quant_wave_one<XDT, CPL, RR, kQuantNone, 64 * CPL, 1>(c, fn, A);     \
    if (f == kQuantW) return quant_wave_one<XDT, CPL, RR, kQuantW, 64 * CPL, 1, false, TL>(c, fn, A);     \
    if (f == kQuantWTab) return quant_wave_one<XDT, CPL, RR, kQuantWTab, 64 * CPL, 1, false, TL>(c, fn, A); \
    if (f == kQuantWTab32) return quant_wave_one<XDT, CPL, RR, kQuantWTab32, 64 * CPL, 1>(c, fn, A); \
    return quant_wave_one<XDT, CPL, RR, kQuantRaw, 64 * CPL, 1>(c, fn, A);
    if (A.rot == H3S_ROT_SYLVESTER && A.group == 128) { H3_QW(rot_with(H3S_ROT_SYLVESTER, 128)) }
    if (A.rot == H3S_ROT_SYLVESTER) { H3_QW(H3S_ROT_SYLVESTER) }
    if (A.rot == H3S_ROT_REGULAR) { H3_QW(H3S_ROT_REGULAR) }
    H3_QW(H3S_ROT_NONE)
#undef H3_QW
}
// The model's own widths (docs/BASELINE.md:13), each with the layout measured fastest for it. With the checkpoints'
// ConvRot group (regular 256), a lane holds 16 consecutive features of a group (two chunks, "pairs"), so every digit
// of the rotation is inside the lane or one DPP operand away; without a rotation, one chunk a lane:
//   5376 features (the hidden width):     the norm with a weight (and float32 tables: the DiT's AdaLN): two
//                                         wavefronts a row, 3 run pairs each, the row's last a quarter full; the
//                                         quantizer on x: one wavefront a row of 6 run pairs, the last a quarter
//                                         full (unrotated: the norm two wavefronts a row of 6 slots, the last of the
//                                         second empty; the quantizer on x one wavefront a row, 11 slots, the last
//                                         half full); with ROW_OUTH h3s_rms_norm_mod itself
//   7168 features (the attention's out):  the quantizer on x: one wavefront a row, 7 run pairs (two wavefronts of
//                                         7 slots unrotated)
//   4096 features:                        the quantizer on x, rotated: two wavefronts a row, two run pairs each
//   8192 features (the MLP's middle of    the quantizer on swiglu(x), rotated: four wavefronts a row, two run pairs
//   the measured 47104 x 8192 workload):  each
//   14336 features (the MLP's middle):    the quantizer on x or on swiglu(x): seven wavefronts a row, two run pairs
//                                         each (four wavefronts of 7 slots unrotated)
template <int XDT> int quant_wave_model(Ctx* c, const char* fn, const QuantArgs& A, int f) {
    const bool reg256 = A.rot == H3S_ROT_REGULAR && A.group == 256, none = A.rot == H3S_ROT_NONE;
    constexpr int R256 = rot_with(H3S_ROT_REGULAR, 256), R0 = H3S_ROT_NONE;
    // the norm (with its side values in LDS) streamed; the quantizers on x or swiglu(x) one row a group
    constexpr int MN = QW_STREAM, MR = QW_ONE;
    if (A.C == 5376) {
        constexpr int N = 672;
        if (f == (kQuantW | ROW_OUTH)) return quant_wave_one<XDT, 6, R0, kQuantW | ROW_OUTH, N, 2, false, 1, MN>(c, fn, A);
        if (f == (kQuantWTab32 | ROW_OUTH)) return quant_wave_one<XDT, 6, R0, kQuantWTab32 | ROW_OUTH, N, 2, false, 1, MN>(c, fn, A);
        if (f == kQuantWTab32 && reg256) return quant_wave_one<XDT, 6, R256, kQuantWTab32, N, 2, true, 1, MN>(c, fn, A);
        if (f == kQuantWTab32 && none) return quant_wave_one<XDT, 6, R0, kQuantWTab32, N, 2, false, 1, MN>(c, fn, A);
        if (f == kQuantW && reg256) return quant_wave_one<XDT, 6, R256, kQuantW, N, 2, true, 1, MN>(c, fn, A);
        if (f == kQuantW && none) return quant_wave_one<XDT, 6, R0, kQuantW, N, 2, false, 1, MN>(c, fn, A);
        if (f == kQuantRaw && reg256) return quant_wave_one<XDT, 12, R256, kQuantRaw, N, 1, true, 1, MR>(c, fn, A);
        if (f == kQuantRaw && none) return quant_wave_one<XDT, 11, R0, kQuantRaw, N, 1, false, 1, MR>(c, fn, A);
    }
    if (A.C == 7168 && f == kQuantRaw) {
        if (reg256) return quant_wave_one<XDT, 14, R256, kQuantRaw, 896, 1, true, 1, MR>(c, fn, A);
        if (none) return quant_wave_one<XDT, 7, R0, kQuantRaw, 896, 2, false, 1, MR>(c, fn, A);
    }
    if (A.C == 4096 && f == kQuantRaw && reg256) return quant_wave_one<XDT, 4, R256, kQuantRaw, 512, 2, true, 1, MR>(c, fn, A);
    if (A.C == 8192 && f == kQuantSwiglu && reg256) return quant_wave_one<XDT, 4, R256, kQuantSwiglu, 1024, 4, true, 1, MR>(c, fn, A);
    if (A.C == 14336) {
        if (f == kQuantRaw && reg256) return quant_wave_one<XDT, 4, R256, kQuantRaw, 1792, 7, true, 1, MR>(c, fn, A);
        if (f == kQuantRaw && none) return quant_wave_one<XDT, 7, R0, kQuantRaw, 1792, 4, false, 1, MR>(c, fn, A);
        if (f == kQuantSwiglu && reg256) return quant_wave_one<XDT, 4, R256, kQuantSwiglu, 1792, 7, true, 1, MR>(c, fn, A);
        if (f == kQuantSwiglu && none) return quant_wave_one<XDT, 7, R0, kQuantSwiglu, 1792, 4, false, 1, MR>(c, fn, A);
    }
    return 1;   // not a shape of this set
}
// whether quant_wave_model takes this call
inline bool quant_wave_model_takes(const QuantArgs& A, int f) {
    const bool reg256 = A.rot == H3S_ROT_REGULAR && A.group == 256, none = A.rot == H3S_ROT_NONE;
    if (f & ROW_OUTH) return A.C == 5376 && none && (f == (kQuantW | ROW_OUTH) || f == (kQuantWTab32 | ROW_OUTH));
    if (!reg256 && !none) return false;
    if (A.C == 5376) return f == kQuantWTab32 || f == kQuantW || f == kQuantRaw;
    if (A.C == 7168) return f == kQuantRaw;
    if (A.C == 4096) return f == kQuantRaw && reg256;
    if (A.C == 8192) return f == kQuantSwiglu && reg256;
    if (A.C == 14336) return f == kQuantRaw || f == kQuantSwiglu;
    return false;
}

// what the quantizer runs on: rms_norm_mod of x, x itself, or swiglu of x; or rms_norm_mod's h itself as the result
enum QuantMode { QUANT_NORM, QUANT_RAW, QUANT_SWIGLU, QUANT_NORM_OUT };

// Launches the kernel for one input type; the plan comes from row_plan.
template <int XDT> int quant_launch(Ctx* c, const char* fn, const QuantArgs& A, int mode, RowPlan p) {
    int f = (A.w ? ROW_W : 0) | (A.scale ? ROW_TAB | (A.tab_dt == H3S_F32 ? ROW_TAB32 : 0) : 0);
    if (XDT == H3S_F32 || A.h_dt != H3S_BF16 || !(f == kQuantNone || f == kQuantW || f == kQuantWTab || f == kQuantWTab32))
        f = ROW_DYN;
    if (mode == QUANT_RAW) f = kQuantRaw;
    if (mode == QUANT_SWIGLU) f = XDT == H3S_F32 || A.h_dt != H3S_BF16 ? (ROW_SWIGLU | ROW_DYN) : kQuantSwiglu;
    if (mode == QUANT_NORM_OUT) f |= ROW_OUTH;
    // the model's widths, one or two wavefronts a row
    if constexpr (XDT != H3S_F32) {
        if (quant_wave_model_takes(A, f) && (A.M >= c->quant_wave_min || (f & ROW_OUTH))) {
            const int r = quant_wave_model<XDT>(c, fn, A, f);
            if (r != 1) return r;
        }
    }
    if (f & ROW_OUTH) return fail(std::string(fn) + ": no kernel stores h for this row shape");
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
