// common.h - what every translation unit of libh3hip.so shares: the context, the error convention, and the
// device-side helpers (element conversions, 16-byte vector access, cross-lane exchanges of a 64-wide wavefront).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/h3hip.h"

#define H3S_EXPORT extern "C" __attribute__((visibility("default")))

namespace h3 {

// ---- host side -------------------------------------------------------------------------------------------------

// the per-thread error message of h3s_last_error (kernels/h3sycl.cpp:40)
void set_error(const std::string& msg);
int fail(const std::string& msg);          // sets the message, returns -1

// The device memory one context answers for. A single budget - H3S_MEM_FRACTION of the card, 0.94 unless set (the
// reference's cap, kernels/h3sycl.cpp:221-224) - covers the caller's buffers (h3s_alloc) and the library's scratch
// regions together. A request that would pass it is refused with the numbers before the driver is asked. Thread-safe.
class Budget {
  public:
    void set_limit(size_t bytes) { std::lock_guard<std::mutex> l(mu_); limit_ = bytes; }
    size_t limit() const { std::lock_guard<std::mutex> l(mu_); return limit_; }
    size_t in_use() const { std::lock_guard<std::mutex> l(mu_); return in_use_; }
    // counts `bytes` more for `what` when they fit; else false, with the refusal as this thread's error
    bool take(size_t bytes, const std::string& what);
    void give_back(size_t bytes) { std::lock_guard<std::mutex> l(mu_); in_use_ -= bytes < in_use_ ? bytes : in_use_; }
    // the caller's buffers: remembered with their size, forgotten (and their bytes given back) when freed
    void remember(void* p, size_t bytes) { std::lock_guard<std::mutex> l(mu_); buffers_[p] = bytes; }
    bool forget(void* p);                               // false when p is not one of the caller's buffers
    std::vector<void*> buffers() const;

  private:
    mutable std::mutex mu_;
    size_t limit_ = 0, in_use_ = 0;
    std::unordered_map<void*, size_t> buffers_;
};

struct Ctx {
    int device = 0;
    hipStream_t stream = nullptr;          // kernels run here, in call order
    bool own_stream = false;
    hipStream_t copy_stream = nullptr;     // h3s_upload, made on first use
    std::mutex copy_mu;
    std::string name;
    int cus = 256;                         // compute units of the device (persistent grids are sized by them)
    bool poison = false;                   // H3S_POISON: fresh buffers filled with 0xff bytes
    Budget budget;
    // The library's scratch: one region per use, kept across calls and grown when a call needs more.
    enum Region {
        LIN_CODES,   // h3s_int8_linear: the int8 rows of a row chunk
        LIN_SCALES,  //   and their row scales
        ATT_Q,       // h3s_attention: q prepared [H, Sp, D] (int8 or half)
        ATT_K,       //   k prepared
        ATT_V,       //   v as half, transposed [H, D, Sp]
        ATT_AUX,     //   the block scales and k's mean
        ATT_PART,    //   the split blocks' partial sums (O, m, l)
        LIN_F32,     // h3s_linear / h3s_linear_acc: the float32 product of a row chunk
        GEMM_PART,   // the matrix-core GEMMs: the accumulators of the split last tiles' parts
        N_REGIONS
    };
    struct Area { void* p = nullptr; size_t bytes = 0; };
    Area areas[N_REGIONS];
    void* blas = nullptr;                  // h3s_linear: the rocBLAS handle, on this context's stream
    bool sage_want = true;                 // H3S_ATTN=onednn: false
    int64_t sage_min_s = 8192;             // H3S_SAGE_MIN_S
    int attn_split = 8;                    // H3S_ATTN_SPLIT: most key ranges a block of a short last round takes (1: none)
    int64_t quant_wave_min = 8192;         // H3S_QUANT_WAVE_MIN_ROWS: fewest rows for the one-wavefront-a-row quantizer
    // H3S_PROFILE (kernels/h3sycl.cpp:117, 228): the int8 linear's time by pass, summed over its row chunks and
    // reported at h3s_destroy; attention's time by phase, reported per call
    bool profile = false;
    double lin_ms[2] = {0.0, 0.0};         // quantize (rotation, row scales and codes in one pass), int8 GEMM
    int64_t lin_chunks = 0;

    // region r with room for at least `bytes`; NULL, with the reason as this thread's error, when it cannot grow
    void* scratch_bytes(Region r, size_t bytes);
    template <typename T> T* scratch(Region r, size_t n) { return static_cast<T*>(scratch_bytes(r, n * sizeof(T))); }
};

// The phases of one call timed with events on the context's stream (H3S_PROFILE): mark() at each boundary, then
// elapsed() waits for the last mark and gives the milliseconds between consecutive marks. Inert when profiling is off.
class PhaseTimer {
  public:
    // allowed false: never times (a caller that must create nothing, h3s_int8_linear_noalloc)
    explicit PhaseTimer(Ctx* c, bool allowed = true);
    ~PhaseTimer();
    void mark();
    std::vector<float> elapsed();
    bool on() const { return on_; }

  private:
    Ctx* c_;
    bool on_;
    std::vector<hipEvent_t> ev_;
};

// one more device allocation, event, stream or library handle made by the library (h3s_alloc_count)
void count_alloc();
// the context of an entry point: NULL with an error when ctx is NULL; makes its device current
Ctx* ctx_of(void* ctx, const char* fn);
// the status of the last launch on this thread, as an error naming fn
int launched(const char* fn);

// frees the context's rocBLAS handle, if it has one (linear.hip)
void release_blas(Ctx* c);
// looks up, once per device, the device address of h3s_int8_linear_noalloc's fixed scratch (int8_gemm.hip); the
// device must be current. 0, or -1 when the lookup failed (the entry point then reports why).
int noalloc_setup(int device);

// the quantizer of h3s_int8_linear (quant.hip): x [M, K] -> regular rotation per group (0: none) -> q, s
int launch_quantize(Ctx* c, const void* x, int x_dt, int64_t M, int64_t K, int group, int8_t* q, float* s);
// h3s_rms_norm_mod on the quantizer's one-wavefront-a-row layout (quant.hip), for the shapes it takes: 0 or -1 when
// it ran, 1 when the shape is not one of them (the row chain kernel then runs it)
int launch_norm_out(Ctx* c, const char* fn, const void* x, int x_dt, int64_t M, int64_t C, const float* w, float eps,
                    const int32_t* rows, const float* scale, const float* shift, void* out, int out_dt);

inline bool aligned16(const void* p) { return ((uintptr_t) p & 15) == 0; }
inline int elem_size(int dt) { return dt == H3S_F32 ? 4 : 2; }
inline bool dt_ok(int dt) { return dt == H3S_F32 || dt == H3S_F16 || dt == H3S_BF16; }
inline int vec_of(int dt) { return 16 / elem_size(dt); }   // elements in one 16-byte vector

// ---- device side -----------------------------------------------------------------------------------------------

constexpr int kWave = 64;

// waits until at most N vector-memory operations of this thread are outstanding (N a constant)
template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// A workgroup barrier that orders LDS only: the LDS accesses before it are complete (lgkmcnt) and no access moves
// across it (the clobber). __syncthreads would also wait for every global load in flight, draining the rows a
// kernel has prefetched at each row statistic.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Orders a wavefront's own LDS accesses: those issued before it are complete, and the compiler moves no memory
// access across it (for an LDS area only this wavefront uses, written by some lanes and read by others).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A value equal on every lane of the wavefront, taken from the first lane: the compiler then keeps it, and what is
// computed from it, in scalar registers (loop control as scalar branches, loads indexed by it as scalar addresses).
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) ((uint64_t) v >> 32));
    return (int64_t) (((uint64_t) hi << 32) | lo);
}

// bf16 <-> f32: widen by shifting; narrow with the hardware's round-to-nearest-even (finite values: the same bits
// as kernels/h3sycl.cpp:42-49; a NaN stays a NaN)
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
// The float32 inputs of a 16-bit rounding are pinned in registers first (an empty asm): the compiler would otherwise
// fold a producing multiply into a mixed-precision fma with one rounding (v_fma_mix), where the arithmetic rounds to
// float32 and then to the 16-bit type.
__device__ __forceinline__ void pin(float& a) { asm volatile("" : "+v"(a)); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    pin(a);
    pin(b);
    f2 v = {a, b};
    bf2 r = __builtin_convertvector(v, bf2);
    uint32_t u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}
__device__ __forceinline__ float round_bf16(float v) { return bf16_lo(pack_bf16(v, 0.0f)); }
__device__ __forceinline__ float f16_lo(uint32_t u) { _Float16 h; uint16_t b = (uint16_t) u; __builtin_memcpy(&h, &b, 2); return (float) h; }
__device__ __forceinline__ float f16_hi(uint32_t u) { return f16_lo(u >> 16); }
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    pin(a);
    pin(b);
    f2 v = {a, b};
    h2 r = __builtin_convertvector(v, h2);          // v_cvt_pk_f16_f32: both halves, round to nearest even
    uint32_t u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}
__device__ __forceinline__ float round_f16(float v) {
    pin(v);
    return (float) (_Float16) v;
}

// a 16-byte vector of element type DT as floats (V = 8 for 16-bit types, 4 for float32)
template <int DT> struct Vec;
template <> struct Vec<H3S_BF16> {
    static constexpr int V = 8;
    __device__ static __forceinline__ void unpack(const uint4& u, float* f) {
        f[0] = bf16_lo(u.x); f[1] = bf16_hi(u.x); f[2] = bf16_lo(u.y); f[3] = bf16_hi(u.y);
        f[4] = bf16_lo(u.z); f[5] = bf16_hi(u.z); f[6] = bf16_lo(u.w); f[7] = bf16_hi(u.w);
    }
    __device__ static __forceinline__ uint4 pack(const float* f) {
        return make_uint4(pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7]));
    }
    __device__ static __forceinline__ float round(float v) { return round_bf16(v); }
};
template <> struct Vec<H3S_F16> {
    static constexpr int V = 8;
    __device__ static __forceinline__ void unpack(const uint4& u, float* f) {
        f[0] = f16_lo(u.x); f[1] = f16_hi(u.x); f[2] = f16_lo(u.y); f[3] = f16_hi(u.y);
        f[4] = f16_lo(u.z); f[5] = f16_hi(u.z); f[6] = f16_lo(u.w); f[7] = f16_hi(u.w);
    }
    __device__ static __forceinline__ uint4 pack(const float* f) {
        return make_uint4(pack_f16(f[0], f[1]), pack_f16(f[2], f[3]), pack_f16(f[4], f[5]), pack_f16(f[6], f[7]));
    }
    __device__ static __forceinline__ float round(float v) { return round_f16(v); }
};
template <> struct Vec<H3S_F32> {
    static constexpr int V = 4;
    __device__ static __forceinline__ void unpack(const uint4& u, float* f) {
        f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y); f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
    }
    __device__ static __forceinline__ uint4 pack(const float* f) {
        return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
    }
    __device__ static __forceinline__ float round(float v) { return v; }
};

// 8 consecutive float32 values (two 16-byte loads) and 8 table values of type TDT
__device__ __forceinline__ void load_f32x(const float* p, float* f, int n) {
#pragma unroll
    for (int k = 0; k < n; k += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + k);
        f[k] = v.x; f[k + 1] = v.y; f[k + 2] = v.z; f[k + 3] = v.w;
    }
}
template <int TDT> __device__ __forceinline__ void load_tab(const void* p, int64_t i, float* f, int n) {
    if constexpr (TDT == H3S_F32) {
        load_f32x((const float*) p + i, f, n);
    } else {
        // n values of a 16-bit table: n / 8 16-byte loads, or one 8-byte load for n = 4
        if (n == 4) {
            const uint2 u = *reinterpret_cast<const uint2*>((const uint16_t*) p + i);
            float g[8];
            Vec<TDT>::unpack(make_uint4(u.x, u.y, 0, 0), g);
            f[0] = g[0]; f[1] = g[1]; f[2] = g[2]; f[3] = g[3];
        } else {
#pragma unroll
            for (int k = 0; k < n; k += 8) Vec<TDT>::unpack(*reinterpret_cast<const uint4*>((const uint16_t*) p + i + k), f + k);
        }
    }
}

// ---- cross-lane exchanges inside a 64-wide wavefront ----
// value of lane (lane ^ OFF). 1, 2: quad permutes; 4: two row shifts, each for half of the lanes; 7: the half-row
// mirror; 8: a row rotate; 16: a swizzle inside each half of the wave; 32: a permute through the LDS crossbar.
template <int OFF> __device__ __forceinline__ float xor_lane(float v) {
    const int x = __float_as_int(v);
    int r;
    if constexpr (OFF == 1) r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);        // quad_perm [1,0,3,2]
    else if constexpr (OFF == 2) r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    else if constexpr (OFF == 4) {
        const int t = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0x5, false);                   // row_shl:4, lanes 0-3, 8-11
        r = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);                             // row_shr:4, lanes 4-7, 12-15
    } else if constexpr (OFF == 7) r = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);  // row_half_mirror
    else if constexpr (OFF == 8) r = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);    // row_ror:8
    else if constexpr (OFF == 16) r = __builtin_amdgcn_ds_swizzle(x, 0x401F);                     // xor 16 within 32
    else {
        static_assert(OFF == 32, "xor_lane: offsets 1..32");
        r = __builtin_amdgcn_ds_bpermute((int) ((__lane_id() ^ 32u) << 2), x);
    }
    return __int_as_float(r);
}

// the canonical butterfly over the lanes of a wave (offsets L/2 .. 1); every lane ends with the same sum. With SW
// the lanes hold their values at the positions l ^ 3 bit2(l) (an involution inside each run of 8 lanes): the
// position's partner 4 away is then the lane 7 away, and the others are unmoved, so the same tree of additions
// over positions is formed.
template <int L, bool SW = false> __device__ __forceinline__ float wave_sum(float s) {
    if constexpr (L >= 64) s = s + xor_lane<32>(s);
    if constexpr (L >= 32) s = s + xor_lane<16>(s);
    if constexpr (L >= 16) s = s + xor_lane<8>(s);
    if constexpr (L >= 8) s = s + xor_lane<SW ? 7 : 4>(s);
    if constexpr (L >= 4) s = s + xor_lane<2>(s);
    if constexpr (L >= 2) s = s + xor_lane<1>(s);
    return s;
}
template <int L> __device__ __forceinline__ float wave_max(float m) {
    if constexpr (L >= 64) m = fmaxf(m, xor_lane<32>(m));
    if constexpr (L >= 32) m = fmaxf(m, xor_lane<16>(m));
    if constexpr (L >= 16) m = fmaxf(m, xor_lane<8>(m));
    if constexpr (L >= 8) m = fmaxf(m, xor_lane<4>(m));
    if constexpr (L >= 4) m = fmaxf(m, xor_lane<2>(m));
    if constexpr (L >= 2) m = fmaxf(m, xor_lane<1>(m));
    return m;
}

// fl(a / 127): Markstein's corrected product with fl(1 / 127), three instructions where the IEEE division takes
// about eleven; equal to the division bit for bit for every non-negative finite float a (checked on gfx950 over all
// of them). For a = +inf the correction's inf - inf would give NaN, so the product itself (inf) is returned, as the
// division gives; NaN stays NaN.
__device__ __forceinline__ float div127(float a) {
    constexpr float r = 1.0f / 127.0f;
    const float q1 = a * r;
    const float q = __builtin_fmaf(__builtin_fmaf(-q1, 127.0f, a), r, q1);
    return q1 == __builtin_inff() ? q1 : q;
}
// 1 / sqrt(mean + eps), each step correctly rounded (built with correctly rounded f32 division and square root)
__device__ __forceinline__ float inv_root(float sum, float n, float eps) { return 1.0f / __builtin_sqrtf(sum / n + eps); }

// rint(y / s) with y / s correctly rounded: q1 = y * r, e = y - q1 * s (exact, one fma), q = q1 + e * r, where
// r = fl(1 / s) is the correctly rounded reciprocal (Markstein's division correction). Then round half to even.
__device__ __forceinline__ float quant_code(float y, float s, float r) {
    const float q1 = y * r;
    const float e = __builtin_fmaf(-q1, s, y);
    const float q = __builtin_fmaf(e, r, q1);
    return fminf(fmaxf(__builtin_rintf(q), -128.0f), 127.0f);
}
// four codes (each in [-128, 127]) as the bytes of one word, lowest first
__device__ __forceinline__ uint32_t pack_i8x4(float a, float b, float c, float d) {
    const uint32_t ia = (uint32_t) (int) a & 0xffu, ib = (uint32_t) (int) b & 0xffu, ic = (uint32_t) (int) c & 0xffu,
                   id = (uint32_t) (int) d & 0xffu;
    return ia | (ib << 8) | (ic << 16) | (id << 24);
}

// pointwise activations (float32): SiLU g / (1 + e^-g) (kernels/h3sycl.cpp:1395); GELU-tanh
// 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))) (engine/h3-core/src/audio.rs:440), evaluated as
// v / (1 + e^(-2u)), u = sqrt(2/pi) (v + 0.044715 v^3), the same function: 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)).
__device__ __forceinline__ float act_silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ __forceinline__ float act_gelu_tanh(float v) {
    // e^(-2u) = 2^(v * (A + B v^2)), A = -2 log2(e) sqrt(2/pi), B = A * 0.044715
    const float A = -2.3022082f, B = -0.10294324f;
    const float e = __builtin_amdgcn_exp2f(v * __builtin_fmaf(B, v * v, A));
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}
template <int ACT> __device__ __forceinline__ float act(float v) {
    if constexpr (ACT == H3S_ACT_SILU) return act_silu(v);
    else if constexpr (ACT == H3S_ACT_GELU_TANH) return act_gelu_tanh(v);
    else return v;
}

}  // namespace h3
