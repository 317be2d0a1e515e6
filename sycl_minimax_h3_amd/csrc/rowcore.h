// rowcore.h - the row layout every per-token row kernel shares, and its canonical reductions.
//
// A token row of C features is cut into 16-byte chunks (V = 8 features of a 16-bit type, 4 of float32). L lanes
// work on one row: lane t holds chunks t, t + L, ..., t + (CPL - 1) L, so each load instruction of a wave covers
// 1 KiB of consecutive bytes. L follows the row length (the oracle's h3o_row_lanes): 64 lanes (one wavefront, four
// rows a 256-thread block) below 256 chunks, 256 lanes (four wavefronts, one row a block) up to 1024 chunks, 512
// lanes (eight wavefronts) up to 2048. CPL = ceil(chunks / L) is at most 4, so every load of a row - the row, the
// residual, the weights and the modulation tables - is issued before the first value is used.
//
// Canonical sums (the oracle's h3o_canon_sum): each lane adds its values in increasing index order, then an xor
// butterfly over the 64 lanes of its wavefront (offsets 32 .. 1); with several wavefronts on the row, their sums go
// through LDS and every wavefront combines them with the same butterfly over wavefront indices. Each butterfly step
// adds the same two values in every lane (a + b = b + a exactly), so all lanes end with identical bits.
#pragma once

#include <algorithm>

#include "common.h"

namespace h3 {

struct RowPlan {
    int L = 0, cpl = 0;
};
// lanes per row and chunks per lane for a row of nch 16-byte chunks; L = 0 when the row is too long
inline RowPlan row_plan(int64_t nch) {
    RowPlan p;
    if (nch <= 0) return p;
    if (nch < 256) { p.L = 64; p.cpl = (int) ((nch + 63) / 64); }
    else if (nch <= 1024) { p.L = 256; p.cpl = (int) ((nch + 255) / 256); }
    else if (nch <= 2048) { p.L = 512; p.cpl = (int) ((nch + 511) / 512); }
    return p;
}
// A launch: 64-lane rows go four to a 256-thread block, wider rows one to a block of L threads.
struct RowLaunch {
    unsigned grid, threads;
    int lshift;                                          // log2 L
};
inline RowLaunch row_launch(int64_t M, RowPlan p) {
    RowLaunch r;
    const int rpb = p.L >= 256 ? 1 : 256 / p.L;
    r.grid = (unsigned) ((M + rpb - 1) / rpb);
    r.threads = (unsigned) (p.L >= 256 ? p.L : 256);
    r.lshift = __builtin_ctz((unsigned) p.L);
    return r;
}
// blocks of a kernel that fit one compute unit at once (with lds bytes of dynamic LDS each), asked of the runtime
// once per kernel, block size and LDS size
int blocks_per_cu(const void* kernel, int threads, size_t lds = 0);

// A launch of row units (blocks of L >= 256 lanes, wavefronts of 64); unit u takes rows [u rpu, (u + 1) rpu). With
// `keep` (side inputs worth holding in registers across rows: table rows) twice as many units as the device holds
// at once, each taking a contiguous run of rows; else one unit a row (measured faster when there is nothing to
// keep). The occupancy of each kernel is asked once.
struct PersistentLaunch {
    unsigned grid, threads;
    int lshift;
    int64_t rpu;                                         // rows a unit
};
inline PersistentLaunch persistent_launch(const Ctx* c, const void* kernel, int64_t M, RowPlan p, bool keep) {
    PersistentLaunch r;
    r.threads = (unsigned) (p.L >= 256 ? p.L : 256);
    r.lshift = __builtin_ctz((unsigned) p.L);
    const int upb = p.L >= 256 ? 1 : 256 / p.L;          // units a block
    const int per_cu = blocks_per_cu(kernel, (int) r.threads);
    const int64_t units = keep ? std::min<int64_t>(M, (int64_t) c->cus * per_cu * upb * 2) : M;
    r.rpu = (M + units - 1) / units;
    const int64_t used = (M + r.rpu - 1) / r.rpu;        // units that get rows
    r.grid = (unsigned) ((used + upb - 1) / upb);
    return r;
}
// where this thread sits: its lane t in the row, and the row (clamped into [0, M); live = false past M)
struct RowPos {
    int t, W;                                            // W: wavefronts on the row
    int64_t row;
    bool live;
};
__device__ __forceinline__ RowPos row_pos(int lshift, int64_t M) {
    RowPos p;
    const int L = 1 << lshift;
    p.t = (int) (threadIdx.x & (L - 1));
    p.W = L >> 6;
    const int64_t r = L >= 256 ? (int64_t) blockIdx.x : (int64_t) blockIdx.x * (256 >> lshift) + (threadIdx.x >> lshift);
    p.live = r < M;
    p.row = p.live ? r : M - 1;
    return p;
}

// The wave sums of one row combined in LDS, each wavefront forming the butterfly over wavefront indices
// (offsets W/2 .. 1); red holds 8 floats and is used by this reduction only.
__device__ __forceinline__ float row_combine_sum(float s, float* red, int W) {
    if (W > 1) {
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        lds_barrier();
        if (W == 4) s = (red[0] + red[2]) + (red[1] + red[3]);
        else s = ((red[0] + red[4]) + (red[2] + red[6])) + ((red[1] + red[5]) + (red[3] + red[7]));
    }
    return s;
}
__device__ __forceinline__ float row_sum(float p, float* red, int W) { return row_combine_sum(wave_sum<64>(p), red, W); }
__device__ __forceinline__ float row_max(float m, float* red, int W) {
    m = wave_max<64>(m);
    if (W > 1) {
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        lds_barrier();
        m = red[0];
        for (int k = 1; k < W; ++k) m = fmaxf(m, red[k]);
    }
    return m;
}

// ---- loads of V values of an element type, issued now and decoded later ----
// WIDE storage holds V float32 values (two 16-byte loads for V = 8, one for V = 4) or V 16-bit ones; narrow storage
// only the 16-bit types (one 16-byte load for V = 8, one 8-byte load for V = 4). The type itself may be a runtime
// value; a constant one folds the branches away.
template <int V, bool WIDE> struct Raw {
    uint4 a;
    uint4 b;                                              // the second half of V = 8 float32 values
};
template <int V> struct Raw<V, false> {
    uint4 a;
};
// Loads of data that is read once (the rows a kernel streams) use the nontemporal form: the lines are not kept for
// reuse. A cold streaming probe (x and a residual read, one output written, 16896 x 4096 bf16 each, over a ring of
// 1.25 GB) moved 73.8 % of 8 TB/s with ordinary loads and 81.3 % with these. Weights and tables, which every row
// reads again, keep ordinary loads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_nt(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_nt2(const void* p) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return make_uint2(v.x, v.y);
}
// NT: a row streamed once (the nontemporal form); else a side input read again by other rows
template <int V, bool WIDE, bool NT = false>
__device__ __forceinline__ void fetch(Raw<V, WIDE>& r, const void* p, int dt, int64_t i) {
    if (WIDE && dt == H3S_F32) {
        const uint4* q = reinterpret_cast<const uint4*>((const float*) p + i);
        r.a = NT ? ld_nt(q) : q[0];
        if constexpr (WIDE && V == 8) r.b = NT ? ld_nt(q + 1) : q[1];
    } else if constexpr (V == 8) {
        const uint4* q = reinterpret_cast<const uint4*>((const uint16_t*) p + i);
        r.a = NT ? ld_nt(q) : *q;
    } else {
        const uint2* q = reinterpret_cast<const uint2*>((const uint16_t*) p + i);
        const uint2 t = NT ? ld_nt2(q) : *q;
        r.a = make_uint4(t.x, t.y, 0u, 0u);
    }
}
template <int V, bool WIDE> __device__ __forceinline__ void decode(const Raw<V, WIDE>& r, int dt, float* f) {
    if (WIDE && dt == H3S_F32) {
        f[0] = __uint_as_float(r.a.x); f[1] = __uint_as_float(r.a.y); f[2] = __uint_as_float(r.a.z); f[3] = __uint_as_float(r.a.w);
        if constexpr (WIDE && V == 8) {
            f[4] = __uint_as_float(r.b.x); f[5] = __uint_as_float(r.b.y); f[6] = __uint_as_float(r.b.z); f[7] = __uint_as_float(r.b.w);
        }
    } else {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        if (dt == H3S_BF16) {
#pragma unroll
            for (int k = 0; k < V / 2; ++k) { f[2 * k] = bf16_lo(w[k]); f[2 * k + 1] = bf16_hi(w[k]); }
        } else {
#pragma unroll
            for (int k = 0; k < V / 2; ++k) { f[2 * k] = f16_lo(w[k]); f[2 * k + 1] = f16_hi(w[k]); }
        }
    }
}

// ---- side inputs of a row kernel: which are present and how wide, fixed at compile time for the call shapes
// that matter for speed; ROW_DYN takes them all at run time (present when non-NULL, float32 or 16-bit) ----
enum : int {
    ROW_W = 1,          // float32 weight [C]
    ROW_B = 2,          // float32 bias [C]
    ROW_TAB = 4,        // scale and shift tables [R, C] (16-bit unless ROW_TAB32)
    ROW_TAB32 = 8,
    ROW_GATE = 16,      // gate table [R, C], the tables' type
    ROW_RES = 32,       // residual [M, C] (16-bit unless ROW_RES32)
    ROW_RES32 = 64,
    ROW_DYN = 128,
    ROW_RAW = 256,      // the quantizer on x itself, with no norm (h3s_int8_linear); no side inputs
    ROW_LN = 512,       // the row chain: layer norm (else RMS norm)
    ROW_ACT1 = 1024,    // the row chain's activation, 2 bits: H3S_ACT_NONE, H3S_ACT_GELU_TANH or H3S_ACT_SILU
    ROW_SWIGLU = 4096,  // the quantizer on silu(gate) * up of a [gate | up] row, with no norm (h3s_swiglu_quant)
    ROW_OUTH = 8192,    // the norm's bfloat16 row h stored as the result, no rotation or codes (h3s_rms_norm_mod)
};
constexpr int row_act(int f) { return (f / ROW_ACT1) & 3; }

// ---- stores that bypass the caches' retention (the outputs are streamed, never read back by the kernel) ----
__device__ __forceinline__ void st_nt(void* p, uint4 v) {
    const u32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void st_nt(void* p, uint2 v) {
    const u32x2 t = {v.x, v.y};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x2*>(p));
}
__device__ __forceinline__ void st_nt(void* p, uint32_t v) { __builtin_nontemporal_store(v, reinterpret_cast<uint32_t*>(p)); }

// V float values stored at element i of out in the runtime type out_dt
template <int V> __device__ __forceinline__ void store_chunk(void* out, int out_dt, int64_t i, const float* f) {
    if (out_dt == H3S_F32) {
        float* o = (float*) out + i;
#pragma unroll
        for (int k = 0; k < V; k += 4)
            st_nt(o + k, make_uint4(__float_as_uint(f[k]), __float_as_uint(f[k + 1]), __float_as_uint(f[k + 2]), __float_as_uint(f[k + 3])));
    } else {
        uint32_t w[V / 2];
        if (out_dt == H3S_BF16) {
#pragma unroll
            for (int k = 0; k < V; k += 2) w[k / 2] = pack_bf16(f[k], f[k + 1]);
        } else {
#pragma unroll
            for (int k = 0; k < V; k += 2) w[k / 2] = pack_f16(f[k], f[k + 1]);
        }
        uint16_t* o = (uint16_t*) out + i;
        if constexpr (V == 8) st_nt(o, make_uint4(w[0], w[1], w[2], w[3]));
        else st_nt(o, make_uint2(w[0], w[1]));
    }
}


}  // namespace h3
