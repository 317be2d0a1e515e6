// gemm_impl.h - the int8 GEMM with the dequant epilogue on gfx950's i8 matrix cores (kernels/h3sycl.cpp:576-631,
// engine/h3-core/src/reference.rs:72-76), used by h3s_int8_linear and h3s_int8_gemm_dequant (int8_gemm.hip); and the
// same pipeline on the bf16 / f16 matrix cores for the float linear (h3s_linear, h3s_linear_acc, linear.hip).
//
//   acc[m, n] = sum_k A[m, k] W[n, k]                    exact int32 (|acc| <= K 128 128 = 2^26 at K = 4096)
//   one weight scale:  v = acc * fl(s[m] * wscale[0])     (the row factor the reference folds first, h3sycl.cpp:576)
//   N weight scales:   v = (acc * s[m]) * wscale[n]       (the post-op order of h3sycl.cpp:588-602)
//   then + bias[n], then the activation, rounded once to out's type.
// 16-bit operands (gemm_f16_kernel): acc in float32 (v_mfma_f32_32x32x16_bf16 / _f16), v = acc [+ bias[n]]
// [+ out[m, n], the old output of h3s_linear_acc], rounded once to out's type (kernels/h3sycl.cpp:656-720). A 32-deep
// int8 slice and a 16-deep 16-bit slice are both 32 bytes of each row, with the same lane layout (lane l: row l % 32,
// bytes 16 (l / 32) .. + 15 of the slice) and the same 32 x 32 accumulator layout, so the operand path below works
// in bytes and serves both: GemmArgs::K is the bytes of a row.
//
// Block: 512 threads (eight wavefronts, 2 x 4, two a SIMD), a 256 x 256 tile of out; each wavefront 128 x 64 as
// 4 x 2 v_mfma_i32_32x32x32_i8 accumulators (128 registers): while one wavefront of a SIMD waits (its fragment reads,
// the step's barrier, its refill loads) the other issues products (four wavefronts of 128 x 128, one a SIMD, ran 6 %
// slower; sixteen of 64 x 64, four a SIMD, 1.5 % slower). K advances 128 bytes a step (four
// 32-deep slices) through two LDS stages (64 KiB each: the A and W rows of the step), filled by direct
// global->LDS loads (global_load_lds_dwordx4), so no registers hold operands in flight; each load instruction reads
// 8 rows x 128 bytes, whole lines (a 64-byte step, half lines per instruction and the other halves a step later,
// measured 4 % slower with four stages). Each step runs its four slices' products with the next slice's fragment
// reads between them, waits for the next stage and publishes it (one barrier), then refills the stage it just
// finished and reads the next stage's first slice, both spread between its last products.
//
// LDS layout of an operand slice: 256 rows x 8 16-byte chunks; chunk c of row r at unit 8 r + (c ^ ((r / 2) % 8)).
// A fragment read (32 consecutive rows, one chunk each) then touches 16 distinct 4-bank groups in each 16-lane
// quarter. The direct loads write 64 consecutive units per instruction, so each lane fetches the (row, chunk) that
// its unit holds: eight lanes cover one row's 128 bytes.
//
// Tile order: the 8 XCDs take blocks round robin; blocks are renumbered so that each XCD works on a contiguous
// run of tiles, grouped 8 tiles high (4 for K of 12288 or more) so that the resident blocks of an XCD share A and W
// panels in its L2.
// Epilogue: per 32-row slice of a wavefront's region, dequant + activation in registers, the slice through LDS,
// then 16-byte row-contiguous stores (h3s_linear_acc: the slice in float32, the old output added as it is stored).
// Split tiles (gemm_plan_split): a short last round of long-K tiles, or every tile of a launch of few tiles, runs
// as several blocks of consecutive K steps that leave their accumulators in scratch; gemm_merge_kernel sums them in
// part order and applies the same epilogue arithmetic (gemm_values).
#pragma once

#include <type_traits>

#include "rowcore.h"

namespace h3 {

constexpr int kGemmBM = 256, kGemmBN = 256, kGemmBK = 128, kGemmStages = 2;
// Each wavefront computes kGemmWM rows x kGemmWN columns of the tile: kGemmWI x kGemmWJ accumulators of 32 x 32,
// kGemmMF products a 32-deep slice, kGemmLoads direct loads of each operand a stage.
constexpr int kGemmWM = 128, kGemmWN = 64, kGemmWI = kGemmWM / 32, kGemmWJ = kGemmWN / 32, kGemmMF = kGemmWI * kGemmWJ;
constexpr int kGemmWaves = (kGemmBM / kGemmWM) * (kGemmBN / kGemmWN), kGemmThreads = 64 * kGemmWaves;
constexpr int kGemmLoads = 32 / kGemmWaves;
constexpr int kGemmStageBytes = (kGemmBM + kGemmBN) * kGemmBK;   // 64 KiB
// the two stages, or the epilogue's scales and per-wavefront 32-row slices of float32 outputs, if larger
constexpr int kGemmEpiBytes = 3 * 1024 + kGemmWaves * 32 * (kGemmWN * 4 + 16);
constexpr int kGemmLds = kGemmStages * kGemmStageBytes > kGemmEpiBytes ? kGemmStages * kGemmStageBytes : kGemmEpiBytes;
constexpr int kGemmTileAcc = kGemmBM * kGemmBN;                   // accumulators of a tile (a split tile's part)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf_g __attribute__((ext_vector_type(8)));
typedef _Float16 v8h_g __attribute__((ext_vector_type(8)));

// the operands' element type: int8 codes (the dequant epilogue) or 16-bit floats (the float epilogue)
enum : int { GEMM_I8 = 0, GEMM_BF16 = 1, GEMM_F16 = 2 };

struct GemmArgs {
    const int8_t* A;          // [M, K] quantized activations (16-bit operands: their bytes)
    const float* sA;          // [M] their scales (NULL for 16-bit operands)
    int64_t M, K;             // K: the bytes of a row (the features for int8, twice them for 16-bit operands)
    const int8_t* W;          // [N, K]
    int64_t N;
    const float* ws;          // [N] or [1] (NULL for 16-bit operands)
    const float* bias;        // [N] or NULL
    void* out;                // [M, N]
    int out_dt;
    int tm, tn;               // tiles along M and N
    int gh;                   // the height of a group of tiles an XCD walks (gemm_tile_of)
    // The last tiles split along K: blocks [0, main_tiles) take tiles 0 .. main_tiles - 1 whole; block main_tiles +
    // u split + p takes part p of tile main_tiles + u (a contiguous share of the K steps) and leaves its
    // accumulators in part[u split + p] (kGemmTileAcc values of 4 bytes, in register order); gemm_merge_kernel then
    // sums each tile's parts in part order and applies the epilogue. split 1: every tile whole.
    int main_tiles, split;
    void* part;
};

__device__ __forceinline__ int gemm_unit(int r, int c) { return (r << 3) | (c ^ ((r >> 1) & 7)); }

// the tile of block b: XCD-contiguous renumbering (the blocks b % 8 = x, which XCD x runs, take the consecutive ids
// x q + min(x, r) + b / 8, q = total / 8, r = total % 8: the first r XCDs one id more), then GH-high groups of tiles
// (GemmArgs::gh: 8, or 4 for the long-K products, whose A and W panels of 256 rows are larger: fc2's K = 14336 at
// 47104 x 5376 took 3.50 against 3.64-3.66 ms with 4, config 5b's K = 4096 2.82 against 2.76-2.80 ms)
__device__ __forceinline__ int gemm_xcd_id(int b, int total) {
    const int q = total / 8, r = total % 8, x = b % 8;
    return x * q + (x < r ? x : r) + b / 8;
}
__device__ __forceinline__ void gemm_tile_of(int id, int tm, int tn, int GH, int* im, int* in) {
    const int group = GH * tn;
    const int first = (id / group) * GH;
    const int rows = tm - first < GH ? tm - first : GH;
    *im = first + (id % group) % rows;
    *in = (id % group) / rows;
}

// A buffer resource over an operand's rows from the tile's first row on, from byte k0 of each row on: reads past the
// matrix's end return zeros. (A function, not a lambda: a lambda returning this type drops the kernel's host stub.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const int8_t* base, int64_t rows_left, int64_t K, int64_t k0) {
    const int64_t n = rows_left * K - k0;
    return __builtin_amdgcn_make_buffer_rsrc((void*) (base + k0), (short) 0, (int) (uint32_t) (n < 0xFFFFFFFFll ? n : 0xFFFFFFFFll),
                                             0x00020000);
}
// a workgroup barrier without the memory fence of __syncthreads (which would wait for every direct load in flight):
// the direct loads a stage needs are waited for explicitly (wait_vm) before it; the clobber keeps the compiler from
// moving LDS accesses across it
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }


// the float32 values of out[m, n .. n + 3] (the old output h3s_linear_acc adds): one vector load where the tile lies
// inside out and its rows start on 16-byte boundaries (n is a multiple of 4), else element by element inside out
template <int OUT>
__device__ __forceinline__ void gemm_old4(const void* out, int64_t m, int64_t n, int64_t M, int64_t N, bool full, float (&o)[4]) {
    if (full) {
        if constexpr (OUT == H3S_F32) {
            const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(out) + m * N + n);
            o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(out) + m * N + n);
            const uint32_t h[2] = {v.x, v.y};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t b = (h[q / 2] >> (16 * (q & 1))) & 0xFFFFu;
                o[q] = OUT == H3S_BF16 ? bf16_lo(b) : f16_lo(b);
            }
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        o[q] = 0.0f;
        if (m < M && n + q < N) {
            const int64_t i = m * N + n + q;
            if constexpr (OUT == H3S_F32) o[q] = reinterpret_cast<const float*>(out)[i];
            else if constexpr (OUT == H3S_BF16) o[q] = bf16_lo(reinterpret_cast<const uint16_t*>(out)[i]);
            else o[q] = f16_lo(reinterpret_cast<const uint16_t*>(out)[i]);
        }
    }
}

// The epilogue's values of out[m][n .. n + 3] from their accumulators a (gemm_body, and gemm_merge_kernel for the split
// tiles: the same roundings in the same order): int8 dequant, acc s[m] wscale[n] or acc f1 with f1 = fl(s[m]
// wscale[0]) (16-bit operands: acc itself), then + bias[n], + the old out (ACC), then the activation
template <int OP, int ACT, bool PER_N, bool BIAS, bool ACC, typename E>
__device__ __forceinline__ void gemm_values(const E (&a)[4], float sr, float f1, const float (&wq)[4], const float (&bq)[4],
                                            const float (&oq)[4], float (&v)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if constexpr (OP != GEMM_I8) v[q] = a[q];
        else if constexpr (PER_N) v[q] = (float) a[q] * sr * wq[q];
        else v[q] = (float) a[q] * f1;
        if constexpr (BIAS) v[q] = v[q] + bq[q];
        if constexpr (ACC) v[q] = v[q] + oq[q];
        v[q] = act<ACT>(v[q]);
    }
}

// The kernel body for the operand type OP; ACC (16-bit operands only): out += the product.
template <int OP, int ACT, bool PER_N, bool ACC>
__device__ __forceinline__ void gemm_body(const GemmArgs& P) {
    static_assert(OP == GEMM_I8 || (ACT == H3S_ACT_NONE && !PER_N), "gemm_body: the float epilogue has no scales or activation");
    static_assert(!ACC || OP != GEMM_I8, "gemm_body: accumulation into out is the float linear's");
    using Acc = std::conditional_t<OP == GEMM_I8, v16i, v16f>;
    __shared__ __attribute__((aligned(16))) int8_t lds[kGemmLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / (kGemmBN / kGemmWN), wn = wave % (kGemmBN / kGemmWN);
    const int64_t K = P.K;
    // K steps of 128 bytes, the last one 64 when K is an odd multiple of 64 (its two slices only); a tile's part
    // runs the steps [kb, ke)
    const int nk = (int) ((K + kGemmBK - 1) / kGemmBK);
    int im, in, kb = 0, ke = nk, part = -1;
    if ((int) blockIdx.x < P.main_tiles) {
        gemm_tile_of(gemm_xcd_id((int) blockIdx.x, P.main_tiles), P.tm, P.tn, P.gh, &im, &in);
    } else {
        const int u = ((int) blockIdx.x - P.main_tiles) / P.split, p = ((int) blockIdx.x - P.main_tiles) % P.split;
        gemm_tile_of(P.main_tiles + u, P.tm, P.tn, P.gh, &im, &in);
        kb = p * nk / P.split;
        ke = (p + 1) * nk / P.split;
        part = u * P.split + p;
    }
    const int64_t m0 = (int64_t) im * kGemmBM, n0 = (int64_t) in * kGemmBN;
    const bool half_last = K % kGemmBK != 0 && ke == nk;
    // Instruction q of wavefront w fills units 64 (4 w + q) .. + 63: rows 8 (4 w + q) + lane / 8, each lane the
    // chunk its unit holds, so one instruction reads 8 whole 128-byte segments. The loads go through buffer resources
    // (gemm_rsrc): rows past the matrix's end read zeros (their products are not stored), so the lanes' 32-bit offsets
    // are the same for both operands and every step, four registers, where clamped 64-bit addresses held 60 more
    // (196 registers against 256 and spills; 2 % faster). A half step's lanes of chunks 4-7 read the next row's first
    // bytes, or zeros after the last row; the slices that would use them are not run.
    uint32_t vo[kGemmLoads];
#pragma unroll
    for (int q = 0; q < kGemmLoads; ++q) {
        const int r = 8 * (kGemmLoads * wave + q) + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
        vo[q] = (uint32_t) (r * K + 16 * c);
    }
    auto issue = [&](int kt) {
        int8_t* st = lds + (kt % kGemmStages) * kGemmStageBytes;
        const int64_t k0 = (int64_t) kt * kGemmBK;
        const __amdgpu_buffer_rsrc_t ra = gemm_rsrc(P.A + m0 * K, P.M - m0, K, k0);
        const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(P.W + n0 * K, P.N - n0, K, k0);
#pragma unroll
        for (int q = 0; q < kGemmLoads; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*) (st + (kGemmLoads * wave + q) * 1024),
                                                     16, vo[q], 0, 0, 0);
#pragma unroll
        for (int q = 0; q < kGemmLoads; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (__attribute__((address_space(3))) void*) (st + kGemmBM * kGemmBK + (kGemmLoads * wave + q) * 1024), 16, vo[q], 0, 0, 0);
    };

    // the epilogue's row and column scales, loaded now (three registers through the K steps) so that their latency
    // is not waited for at the end
    float sv = 0.0f, wv = 0.0f, bv = 0.0f;
    if (tid < kGemmBM) {
        const int64_t m = m0 + tid < P.M ? m0 + tid : P.M - 1, n = n0 + tid < P.N ? n0 + tid : P.N - 1;
        if constexpr (OP == GEMM_I8) sv = P.sA[m];
        if constexpr (PER_N) wv = P.ws[n];
        if (P.bias) bv = P.bias[n];
    }

    Acc acc[kGemmWI][kGemmWJ];
#pragma unroll
    for (int i = 0; i < kGemmWI; ++i)
#pragma unroll
        for (int j = 0; j < kGemmWJ; ++j) acc[i][j] = (Acc) 0;

    // fragment bases (bytes in a stage) of slice kk: row l % 32 of the wavefront's first 32-row tile, chunk
    // 2 kk + l / 32; tile i is 4096 i further (32 rows of 128 bytes, the swizzle the same for every tile)
    int offA[4], offW[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int c = 2 * kk + (lane >> 5);
        offA[kk] = gemm_unit(wm * kGemmWM + (lane & 31), c) * 16;
        offW[kk] = kGemmBM * kGemmBK + gemm_unit(wn * kGemmWN + (lane & 31), c) * 16;
    }

    // the fragments of one 32-deep slice kk of stage kt (kGemmWI of A and kGemmWJ of W)
    auto read_half = [&](int kt, int kk, v4i (&a)[kGemmWI], v4i (&b)[kGemmWJ]) {
        const int8_t* st = lds + (kt % kGemmStages) * kGemmStageBytes;
#pragma unroll
        for (int i = 0; i < (kGemmWI > kGemmWJ ? kGemmWI : kGemmWJ); ++i) {
            if (i < kGemmWI) a[i] = *reinterpret_cast<const v4i*>(st + offA[kk] + 4096 * i);
            if (i < kGemmWJ) b[i] = *reinterpret_cast<const v4i*>(st + offW[kk] + 4096 * i);
        }
    };
    // W's fragment as the first operand: acc[i][j] holds rows (columns of out) from W tile j and columns (rows of
    // out) from A tile i, so each lane ends with four consecutive output columns of one output row per register group
    auto mfma = [&](const v4i (&a)[kGemmWI], const v4i (&b)[kGemmWJ], int p) {
        const int i = p / kGemmWJ, j = p % kGemmWJ;
        if constexpr (OP == GEMM_I8) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[j], a[i], acc[i][j], 0, 0, 0);
        else if constexpr (OP == GEMM_BF16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_g, b[j]), __builtin_bit_cast(v8bf_g, a[i]),
                                                                acc[i][j], 0, 0, 0);
        else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_g, b[j]), __builtin_bit_cast(v8h_g, a[i]),
                                                               acc[i][j], 0, 0, 0);
    };
    int issued = kb;
    for (; issued < kb + kGemmStages && issued < ke; ++issued) issue(issued);
    v4i xa[kGemmWI], xb[kGemmWJ], ya[kGemmWI], yb[kGemmWJ];
    if (issued - kb > 1) wait_vm<2 * kGemmLoads>(); else wait_vm<0>();
    block_barrier();
    read_half(kb, 0, xa, xb);
    // a slice's products (kGemmMF) with the next slice's fragment reads (kGemmWI + kGemmWJ) between them
    auto body16 = [&](const v4i (&a)[kGemmWI], const v4i (&b)[kGemmWJ]) {
        constexpr int NR = kGemmWI + kGemmWJ;
#pragma unroll
        for (int p = 0; p < kGemmMF; ++p) mfma(a, b, p);
#pragma unroll
        for (int g = 0; g < (NR < kGemmMF ? NR : kGemmMF); ++g) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x0100, NR <= kGemmMF ? 1 : (NR + kGemmMF - 1) / kGemmMF, 0);
        }
        if constexpr (kGemmMF > NR) __builtin_amdgcn_sched_group_barrier(0x0008, kGemmMF - NR, 0);
    };
    // a step with the refill of stage kt + 2 (all but the last two steps) or without it, so that the loads sit in
    // the same scheduling region as the products they are interleaved with
    auto step = [&](int kt, auto refill_tag) {
        constexpr bool REFILL = decltype(refill_tag)::value;
        read_half(kt, 1, ya, yb);
        body16(xa, xb);
        read_half(kt, 2, xa, xb);
        body16(ya, yb);
        read_half(kt, 3, ya, yb);
        body16(xa, xb);
        constexpr int PRE = kGemmMF / 4;      // the last slice's products before the barrier
#pragma unroll
        for (int p = 0; p < PRE; ++p) mfma(ya, yb, p);
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        wait_vm<0>();                         // stage kt + 1 landed (the only one in flight)
        block_barrier();
        if constexpr (REFILL) issue(kt + 2);
        read_half(kt + 1, 0, xa, xb);
#pragma unroll
        for (int p = PRE; p < kGemmMF; ++p) mfma(ya, yb, p);
        // the rest of the slice's products, with the refill loads and the next stage's first fragment reads between them
        if constexpr (REFILL) {
#pragma unroll
            for (int g = 0; g < kGemmMF - PRE; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x0020, (2 * kGemmLoads + kGemmMF - PRE - 1) / (kGemmMF - PRE), 0);
                __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);
            }
        } else {
#pragma unroll
            for (int g = 0; g < kGemmMF - PRE; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);
            }
        }
    };
    int kt = kb;
    for (; kt < ke - 2; ++kt) step(kt, std::true_type{});
    for (; kt < ke - 1; ++kt) step(kt, std::false_type{});
    // the last step: no stage after it; a half step has slices 0 and 1 only
    read_half(ke - 1, 1, ya, yb);
    body16(xa, xb);
    if (!half_last) {
        read_half(ke - 1, 2, xa, xb);
        body16(ya, yb);
        read_half(ke - 1, 3, ya, yb);
        body16(xa, xb);
    }
#pragma unroll
    for (int p = 0; p < kGemmMF; ++p) mfma(ya, yb, p);
    wait_vm<0>();
    if (part >= 0) {
        // a part of a split tile: its accumulators, register by register, 64 lanes' 4-byte values contiguous
        using E = std::conditional_t<OP == GEMM_I8, int, float>;
        // (the 32 x 32 blocks wholly past out's last row or column are not stored: the merge reads none of them)
        E* dst = reinterpret_cast<E*>(P.part) + (size_t) part * kGemmTileAcc + wave * (kGemmMF * 16 * 64) + lane;
#pragma unroll
        for (int i = 0; i < kGemmWI; ++i)
#pragma unroll
            for (int j = 0; j < kGemmWJ; ++j) {
                if (m0 + wm * kGemmWM + 32 * i >= P.M || n0 + wn * kGemmWN + 32 * j >= P.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) dst[((i * kGemmWJ + j) * 16 + r) * 64] = acc[i][j][r];
            }
        return;
    }
    __syncthreads();   // every stage read: the LDS is the epilogue's now

    // ---- epilogue ----
    // Register r of acc[i][j] holds out[m][n] with m = wm 128 + 32 i + lane % 32 and
    // n = wn 64 + 32 j + 8 (r / 4) + 4 (lane / 32) + r % 4: four consecutive columns per group of four registers.
    // Per 32-row slice i of this wavefront's 128 x 64 region: dequant + activation in registers, the four columns
    // as one 8-byte (16-bit out) or 16-byte (float32 out) LDS write, then 16-byte row-contiguous global stores.
    // One wavefront writes and reads its own slice, and a wavefront's LDS operations run in order.
    float* srow = reinterpret_cast<float*>(lds);            // s[m] of the block's 256 rows
    float* wcol = srow + kGemmBM;                           // wscale[n] of its 256 columns
    float* bcol = wcol + kGemmBN;                           // bias[n]
    if (tid < kGemmBM) {
        srow[tid] = sv;
        wcol[tid] = wv;
        bcol[tid] = bv;
    }
    __syncthreads();
    auto epilogue = [&](auto out_tag, auto bias_tag) {
        constexpr int OUT = decltype(out_tag)::value;
        constexpr bool BIAS = decltype(bias_tag)::value;
        constexpr int esz = OUT == H3S_F32 ? 4 : 2;
        // h3s_linear_acc (ACC) stages the values unrounded, as float32, and adds the old output where it stores them:
        // the old rows are then read as whole 16-byte pieces beside the stores
        constexpr int sesz = ACC ? 4 : esz;
        constexpr int pitch = kGemmWN * sesz + 16;          // bytes a slice row (16 bytes of pad: distinct banks)
        int8_t* slice = lds + 3 * 1024 + wave * (32 * pitch);
        const float ws0 = OP == GEMM_I8 && !PER_N ? P.ws[0] : 0.0f;
        // rows of out start on 16-byte boundaries and the block's tile lies inside out: plain 16-byte stores
        const bool full = (P.N * esz) % 16 == 0 && m0 + kGemmBM <= P.M && n0 + kGemmBN <= P.N;
        constexpr int per_row = kGemmWN * esz / 16, epc = 16 / esz, kpl = 32 * per_row / 64;
        // h3s_linear_acc on a tile inside out: the old output of a slice's pieces loaded a slice ahead (slice 0's
        // before any arithmetic), so their latency passes under a slice's work instead of stalling its stores
        uint4 oldv[2][ACC ? kpl : 1];
        auto load_old = [&](int i, uint4 (&d)[ACC ? kpl : 1]) {
#pragma unroll
            for (int k = 0; k < kpl; ++k) {
                const int ch = lane + 64 * k, rr = ch / per_row, cg = ch % per_row;
                const int64_t m = m0 + wm * kGemmWM + i * 32 + rr, n = n0 + wn * kGemmWN + (int64_t) cg * epc;
                d[k] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(P.out) + (m * P.N + n) * esz);
            }
        };
        if constexpr (ACC) {
            if (full) load_old(0, oldv[0]);
        }
#pragma unroll
        for (int i = 0; i < kGemmWI; ++i) {
            const float sr = srow[wm * kGemmWM + i * 32 + (lane & 31)];
            const float f1 = sr * ws0;
#pragma unroll
            for (int j = 0; j < kGemmWJ; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int cl = wn * kGemmWN + j * 32 + 8 * g + 4 * (lane >> 5);    // first of the four columns
                    using E = std::conditional_t<OP == GEMM_I8, int, float>;
                    const E a[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                    float wq[4] = {0.0f, 0.0f, 0.0f, 0.0f}, bq[4] = {0.0f, 0.0f, 0.0f, 0.0f}, oq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (PER_N) {
                        const float4 w4 = *reinterpret_cast<const float4*>(wcol + cl);
                        wq[0] = w4.x; wq[1] = w4.y; wq[2] = w4.z; wq[3] = w4.w;
                    }
                    if constexpr (BIAS) {
                        const float4 b4 = *reinterpret_cast<const float4*>(bcol + cl);
                        bq[0] = b4.x; bq[1] = b4.y; bq[2] = b4.z; bq[3] = b4.w;
                    }
                    float v[4];
                    gemm_values<OP, ACT, PER_N, BIAS, false>(a, sr, f1, wq, bq, oq, v);
                    int8_t* at = slice + (lane & 31) * pitch + (j * 32 + 8 * g + 4 * (lane >> 5)) * sesz;
                    if constexpr (OUT == H3S_F32 || ACC)
                        *reinterpret_cast<float4*>(at) = make_float4(v[0], v[1], v[2], v[3]);
                    else if constexpr (OUT == H3S_BF16)
                        *reinterpret_cast<uint2*>(at) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
                    else
                        *reinterpret_cast<uint2*>(at) = make_uint2(pack_f16(v[0], v[1]), pack_f16(v[2], v[3]));
                }
            const int64_t mt = m0 + wm * kGemmWM + i * 32, nt = n0 + wn * kGemmWN;
            if constexpr (ACC) {
                if (full && i + 1 < kGemmWI) load_old(i + 1, oldv[(i + 1) & 1]);
                // each 16-byte piece of a row of out: its epc staged values + the old ones, rounded once
#pragma unroll
                for (int k = 0; k < kpl; ++k) {
                    const int ch = lane + 64 * k, rr = ch / per_row, cg = ch % per_row;
                    const int64_t m = mt + rr, n = nt + (int64_t) cg * epc;
                    float f[epc];
#pragma unroll
                    for (int q = 0; q < epc; q += 4) {
                        const float4 t = *reinterpret_cast<const float4*>(slice + rr * pitch + (cg * epc + q) * 4);
                        f[q] = t.x; f[q + 1] = t.y; f[q + 2] = t.z; f[q + 3] = t.w;
                    }
                    char* o = reinterpret_cast<char*>(P.out) + (m * P.N + n) * esz;
                    if (full) {
                        const uint4 old = oldv[i & 1][k];
                        const uint32_t w4[4] = {old.x, old.y, old.z, old.w};
                        uint32_t r4[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            if constexpr (OUT == H3S_F32) r4[q] = __float_as_uint(f[q] + __uint_as_float(w4[q]));
                            else if constexpr (OUT == H3S_BF16) r4[q] = pack_bf16(f[2 * q] + bf16_lo(w4[q]), f[2 * q + 1] + bf16_hi(w4[q]));
                            else r4[q] = pack_f16(f[2 * q] + f16_lo(w4[q]), f[2 * q + 1] + f16_hi(w4[q]));
                        }
                        st_nt(o, make_uint4(r4[0], r4[1], r4[2], r4[3]));
                    } else if (m < P.M && n < P.N) {
                        for (int e = 0; e < epc && n + e < P.N; ++e) {
                            if constexpr (OUT == H3S_F32) reinterpret_cast<float*>(o)[e] = f[e] + reinterpret_cast<const float*>(o)[e];
                            else if constexpr (OUT == H3S_BF16)
                                reinterpret_cast<uint16_t*>(o)[e] = (uint16_t) pack_bf16(f[e] + bf16_lo(reinterpret_cast<const uint16_t*>(o)[e]), 0.0f);
                            else
                                reinterpret_cast<uint16_t*>(o)[e] = (uint16_t) pack_f16(f[e] + f16_lo(reinterpret_cast<const uint16_t*>(o)[e]), 0.0f);
                        }
                    }
                }
                continue;
            }
#pragma unroll
            for (int k = 0; k < 32 * per_row / 64; ++k) {
                const int ch = lane + 64 * k, rr = ch / per_row, cg = ch % per_row;
                const int64_t m = mt + rr, n = nt + (int64_t) cg * epc;
                const uint4 val = *reinterpret_cast<const uint4*>(slice + rr * pitch + cg * 16);
                char* o = reinterpret_cast<char*>(P.out) + (m * P.N + n) * esz;
                if (full) {
                    st_nt(o, val);
                } else if (m < P.M && n < P.N) {
                    const uint32_t w4[4] = {val.x, val.y, val.z, val.w};
                    for (int e = 0; e < epc && n + e < P.N; ++e) {
                        if constexpr (esz == 4) reinterpret_cast<uint32_t*>(o)[e] = w4[e];
                        else reinterpret_cast<uint16_t*>(o)[e] = (uint16_t) (w4[e / 2] >> (16 * (e & 1)));
                    }
                }
            }
        }
    };
    using bf16_t = std::integral_constant<int, H3S_BF16>;
    using f16_t = std::integral_constant<int, H3S_F16>;
    using f32_t = std::integral_constant<int, H3S_F32>;
    using yes = std::true_type;
    using no = std::false_type;
    if (P.out_dt == H3S_BF16) { if (P.bias) epilogue(bf16_t{}, yes{}); else epilogue(bf16_t{}, no{}); }
    else if (P.out_dt == H3S_F16) { if (P.bias) epilogue(f16_t{}, yes{}); else epilogue(f16_t{}, no{}); }
    else { if (P.bias) epilogue(f32_t{}, yes{}); else epilogue(f32_t{}, no{}); }
}

template <int ACT, bool PER_N>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_i8_kernel(GemmArgs P) {
    gemm_body<GEMM_I8, ACT, PER_N, false>(P);
}
// the float linear: 16-bit operands (OP GEMM_BF16 or GEMM_F16), out = x w^T [+ bias] (ACC: out += x w^T [+ bias])
template <int OP, bool ACC>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_f16_kernel(GemmArgs P) {
    gemm_body<OP, H3S_ACT_NONE, false, ACC>(P);
}

// The split tiles' epilogue: a thread takes one group of four accumulators of a tile (the wavefront, 32 x 32 block,
// register group and lane of the part layout), sums the tile's parts in part order (int32: exact, the whole tile's
// sum; float32: a fixed order), then the epilogue of gemm_body on out[m][n .. n + 3]. 64 blocks of 256 a tile.
constexpr int kGemmMergeBlocks = kGemmTileAcc / 4 / 256;
template <int OP, int ACT, bool PER_N, bool ACC, int OUT, bool BIAS>
__global__ __launch_bounds__(256) void gemm_merge_kernel(GemmArgs P) {
    using E = std::conditional_t<OP == GEMM_I8, int, float>;
    const int u = (int) blockIdx.x / kGemmMergeBlocks;
    const int t = ((int) blockIdx.x % kGemmMergeBlocks) * 256 + (int) threadIdx.x;
    const int lane = t & 63, grp = t >> 6;              // grp = ((wave kGemmWI + i) kGemmWJ + j) 4 + g
    const int g = grp & 3, j = (grp >> 2) % kGemmWJ, i = (grp >> 2) / kGemmWJ % kGemmWI, wave = (grp >> 2) / kGemmMF;
    const int wm = wave / (kGemmBN / kGemmWN), wn = wave % (kGemmBN / kGemmWN);
    int im, in;
    gemm_tile_of(P.main_tiles + u, P.tm, P.tn, P.gh, &im, &in);
    const int64_t m = (int64_t) im * kGemmBM + wm * kGemmWM + i * 32 + (lane & 31);
    const int64_t n = (int64_t) in * kGemmBN + wn * kGemmWN + j * 32 + 8 * g + 4 * (lane >> 5);
    if (m >= P.M || n >= P.N) return;
    const E* src = reinterpret_cast<const E*>(P.part) + (size_t) u * P.split * kGemmTileAcc +
                   ((wave * kGemmWI + i) * kGemmWJ + j) * 16 * 64 + 4 * g * 64 + lane;
    E a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = src[q * 64];
    for (int p = 1; p < P.split; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] = a[q] + src[(size_t) p * kGemmTileAcc + q * 64];
    float sr = 0.0f, f1 = 0.0f, wq[4] = {0.0f, 0.0f, 0.0f, 0.0f}, bq[4] = {0.0f, 0.0f, 0.0f, 0.0f}, oq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (OP == GEMM_I8) {
        sr = P.sA[m];
        if constexpr (!PER_N) f1 = sr * P.ws[0];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t nq = n + q < P.N ? n + q : P.N - 1;
        if constexpr (PER_N) wq[q] = P.ws[nq];
        if constexpr (BIAS) bq[q] = P.bias[nq];
    }
    if constexpr (ACC) gemm_old4<OUT>(P.out, m, n, P.M, P.N, false, oq);
    float v[4];
    gemm_values<OP, ACT, PER_N, BIAS, ACC>(a, sr, f1, wq, bq, oq, v);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (n + q >= P.N) break;
        const int64_t at = m * P.N + n + q;
        if constexpr (OUT == H3S_F32) reinterpret_cast<float*>(P.out)[at] = v[q];
        else if constexpr (OUT == H3S_BF16) reinterpret_cast<uint16_t*>(P.out)[at] = (uint16_t) pack_bf16(v[q], 0.0f);
        else reinterpret_cast<uint16_t*>(P.out)[at] = (uint16_t) pack_f16(v[q], 0.0f);
    }
}

// How the tiles of a launch split (host side): for rows of at least 12288 bytes (96 K steps), when the tiles leave a
// last round of the device (one block a CU) at most half full, each of those tiles becomes `split` blocks of
// consecutive K steps (at most 8, at least 2 steps each, and no more blocks than CUs); the rest run whole. The last
// round runs faster than a full one (fewer CUs draw power: the clock rises), so what a split saves is about 0.4 of
// the round's share it removes, and the merge costs about 15 us: fc2's 1386 tiles at 16896 x 14336 -> 5376 took
// 1191-1194 against 1211-1221 us (2 parts), 3864 at 47104 tokens 3258-3261 against 3322 us (8 parts); with 7168-byte
// rows, 16896 tokens lost 1.5 % (622 against 608-618 us) and 47104 gained 1 %.
// A launch of at most half as many tiles as CUs (a narrow product: a LoRA's first factor, 16896 x 5376 -> 64, is 66
// tiles) splits every tile the same way, where that pays: there the split spreads one round's work over more CUs
// instead of shortening a last round. A tile takes about 1.2 us a K step and a merge about 3 us plus 0.05 us a part
// (its 256 KiB written and read), so the split is taken when 1.2 nk (1 - 1/s) > 0.05 T s + 3 (T tiles, s parts).
inline void gemm_plan_split(int64_t tiles, int64_t nk, int cus, int* main_tiles, int* split) {
    *main_tiles = (int) tiles;
    *split = 1;
    const int64_t full = tiles / cus * cus, rem = tiles - full;
    const bool narrow = full == 0 && 2 * rem <= cus;
    if (!narrow && (nk < 96 || rem == 0 || 2 * rem > cus)) return;
    int64_t s = cus / rem;
    s = s < 8 ? s : 8;
    s = s < nk / 2 ? s : nk / 2;
    if (s < 2) return;
    if (narrow && 24 * nk * (s - 1) <= rem * s * s + 60 * s) return;
    *main_tiles = (int) full;
    *split = (int) s;
}

}  // namespace h3
