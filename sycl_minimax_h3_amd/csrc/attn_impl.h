// attn_impl.h - attention on gfx950's matrix cores: out = softmax(q k^T / sqrt(D)) v per head (kernels/h3sycl.h:185-192),
// in the reference's two forms (kernels/h3sycl.cpp:1676-1767 and 1496-1550):
//   SAGE:  q and k - mean(k) as int8 with one scale per head per 64 rows (the preparation kernels below restate the
//          reference's quantization exactly), scores on the i8 matrix cores, exact in int32;
//   16-bit: q and k in IEEE half, scores on the f16 matrix cores with float32 accumulation.
// Both: v in IEEE half, the softmax online in float32 (base 2), P in half, P v on the f16 matrix cores, the result
// divided by the row sum, rounded to half (the reference's result buffer is half) and stored in out's type.
//
// Layouts (prepared once per call, in the context's scratch): codes or halves of q and k [H, Sp, DK], v transposed to
// half [H, DK, Sp], Sp = S rounded up to 128 with zero rows, DK = the head size D rounded up to 64, 128 or 256 with zero
// features (which change no score and no block max); the output keeps the D features. One block = 4 wavefronts = 128 queries of one head; a
// wavefront owns 32 queries and walks all keys 64 at a time. Per 64-key tile:
//   S^T = K Q^T:  v_mfma_i32_32x32x32_i8 (or f32_32x32x16_f16) with K as the first operand, so every lane ends with
//                 scores of one query (lane % 32) for 32 of the 64 keys (the other 32 in lane ^ 32);
//   softmax:      the row max needs one exchange with lane ^ 32 (v_permlane32_swap); the exponents' reference
//                 point moves only when a tile max passes it by 2^8; the row sum stays a per-lane partial until the end;
//   O^T += V^T P^T: v_mfma_f32_32x32x16_f16 with V^T as the first operand; P's registers become the second operand
//                 after one v_permlane32_swap per register pair (each lane then holds 8 consecutive keys).
// K and V^T tiles go global -> LDS by direct loads (global_load_lds_dwordx4) into two stages, the next tile in flight
// while this one is computed. Tile rows are R bytes long (R / 16 chunks); chunk c of row r sits at chunk
// c ^ ((r / max(1, 16 / (R / 16))) % (R / 16)) of its row, so the 16-byte fragment reads of 16 consecutive rows hit
// distinct banks.
#pragma once

#include <type_traits>

#include "rowcore.h"

namespace h3 {

typedef int v4i_a __attribute__((ext_vector_type(4)));
typedef int v16i_a __attribute__((ext_vector_type(16)));
typedef float v16f_a __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_a __attribute__((ext_vector_type(8)));
typedef _Float16 h2_a __attribute__((ext_vector_type(2)));
constexpr h2_a h2_one = {(_Float16) 1.0f, (_Float16) 1.0f};

constexpr int kAttnRows = 64;            // the reference's scale block (kSageBlock, h3sycl.cpp:1681) and the key tile
constexpr int kAttnQBlock = 128;         // queries of a block
constexpr int kAttnMaxD = 256;           // the largest head: heads of D features run in kernels of 64, 128 or 256
// the kernel head size of a head of D features (D <= kAttnMaxD)
inline int attn_dk(int64_t D) { return D <= 64 ? 64 : D <= 128 ? 128 : 256; }

// ---- preparation ----
template <int DT> __device__ __forceinline__ float attn_elem(const void* p, int64_t i) {
    if constexpr (DT == H3S_F32) return ((const float*) p)[i];
    else if constexpr (DT == H3S_BF16) return bf16_lo(((const uint16_t*) p)[i]);
    else return f16_lo(((const uint16_t*) p)[i]);
}
__device__ __forceinline__ uint16_t half_bits(float x) {
    _Float16 h = (_Float16) x;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

// k's mean over the sequence per (head, feature): a float32 sum in token order, / S (h3sycl.cpp:1732-1737). Each
// feature's sum is one serial chain of S additions, so the kernel is built to run that chain at the adder's latency:
// a block takes 32 features (128 blocks at 4096 features). Wavefronts 1-3 fill a ring of four 12 KiB row chunks with
// direct loads (global_load_lds_dwordx4, three chunks in flight); wavefront 0 runs the 32 sums, one feature a lane,
// with ordinary LDS reads 16 rows ahead of the additions. Wavefront 0 issues no global loads, so the waits the
// compiler places before its LDS reads are exact and never wait on the ring's loads. Needs the rows 16-byte aligned
// (k and the stride); attn_kmean_rows_kernel is the general form.
constexpr int kKmeanFeat = 32, kKmeanStages = 4, kKmeanChunk = 12288, kKmeanLoaders = 192;
template <int DT>
__global__ __launch_bounds__(256) void attn_kmean_kernel(const void* __restrict__ k, int64_t S, int64_t stride,
                                                         float* __restrict__ mean) {
    constexpr int ESZ = DT == H3S_F32 ? 4 : 2, RB = kKmeanFeat * ESZ;          // bytes of a row's 32 features
    constexpr int SEG = RB / 16, ROWS = kKmeanChunk / RB, LPT = kKmeanChunk / (kKmeanLoaders * 16);
    static_assert(kKmeanChunk % RB == 0 && kKmeanChunk % (kKmeanLoaders * 16) == 0, "attn_kmean_kernel: chunk shape");
    __shared__ __attribute__((aligned(16))) uint8_t ring[kKmeanStages * kKmeanChunk];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t c0 = (int64_t) blockIdx.x * kKmeanFeat, nch = (S + ROWS - 1) / ROWS;
    const char* base = reinterpret_cast<const char*>(k) + c0 * ESZ;
    // loader thread p = tid - 64, load i: unit u = p + 192 i of the chunk (row u / SEG, 16-byte segment u % SEG),
    // landing at byte 16 u of the stage: the chunk is row-major, RB bytes a row
    auto issue = [&](int64_t ch) {
        uint8_t* st = ring + (ch % kKmeanStages) * kKmeanChunk;
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int u = (tid - 64) + kKmeanLoaders * i;
            int64_t row = ch * ROWS + u / SEG;
            row = row < S ? row : S - 1;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*) (base + row * stride * ESZ + 16 * (u % SEG)),
                                             (__attribute__((address_space(3))) void*) (st + (3 * i + wave - 1) * 1024), 16, 0, 0);
        }
    };
    // the value of row r of a stage for this lane's feature, as float32
    auto at = [&](const uint8_t* st, int r) -> float {
        const uint8_t* e = st + r * RB + lane * ESZ;
        if constexpr (DT == H3S_F32) return *reinterpret_cast<const float*>(e);
        else if constexpr (DT == H3S_BF16) return bf16_lo(*reinterpret_cast<const uint16_t*>(e));
        else return f16_lo(*reinterpret_cast<const uint16_t*>(e));
    };
    float sum = 0.0f;
    if (wave > 0)
        for (int64_t ch = 0; ch < kKmeanStages - 1 && ch < nch; ++ch) issue(ch);
    for (int64_t ch = 0; ch < nch; ++ch) {
        if (wave > 0) {
            // this chunk has landed once the loads of the (at most two) chunks issued after it are all that is left
            const int64_t after = (nch - 1 - ch) < kKmeanStages - 2 ? nch - 1 - ch : kKmeanStages - 2;
            if (after >= 2) wait_vm<2 * LPT>();
            else if (after == 1) wait_vm<LPT>();
            else wait_vm<0>();
        }
        lds_barrier();                       // chunk ch is in; wavefront 0's reads of chunk ch - 1 are complete
        if (wave > 0 && ch + kKmeanStages - 1 < nch) issue(ch + kKmeanStages - 1);   // into chunk ch - 1's stage
        if (wave == 0 && lane < kKmeanFeat) {
            const uint8_t* st = ring + (ch % kKmeanStages) * kKmeanChunk;
            const int rows = S - ch * ROWS < ROWS ? (int) (S - ch * ROWS) : ROWS;
            const int full = rows / 16 * 16;
            float va[16], vb[16];
            if (full > 0)
#pragma unroll
                for (int i = 0; i < 16; ++i) va[i] = at(st, i);
            for (int r = 0; r < full; r += 32) {
                const bool b1 = r + 16 < full, b2 = r + 32 < full;
                if (b1)
#pragma unroll
                    for (int i = 0; i < 16; ++i) vb[i] = at(st, r + 16 + i);
#pragma unroll
                for (int i = 0; i < 16; ++i) sum = sum + va[i];
                if (b1) {
                    if (b2)
#pragma unroll
                        for (int i = 0; i < 16; ++i) va[i] = at(st, r + 32 + i);
#pragma unroll
                    for (int i = 0; i < 16; ++i) sum = sum + vb[i];
                }
            }
            for (int r = full; r < rows; ++r) sum = sum + at(st, r);
        }
    }
    if (wave == 0 && lane < kKmeanFeat) mean[c0 + lane] = sum / (float) S;
}
// the same sums with element loads, for rows that are not 16-byte aligned
template <int DT>
__global__ __launch_bounds__(256) void attn_kmean_rows_kernel(const void* __restrict__ k, int64_t S, int64_t HD, int64_t stride,
                                                              float* __restrict__ mean) {
    const int64_t hd = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (hd >= HD) return;
    float sum = 0.0f;
    int64_t t = 0;
    for (; t + 8 <= S; t += 8) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = attn_elem<DT>(k, (t + i) * stride + hd);
#pragma unroll
        for (int i = 0; i < 8; ++i) sum = sum + x[i];
    }
    for (; t < S; ++t) sum = sum + attn_elem<DT>(k, t * stride + hd);
    mean[hd] = sum / (float) S;
}

// q or k (- mean) of one head and 64 rows: SAGE to int8 codes with the block's scale (h3sycl.cpp:1735-1754), else to
// half; rows past S become zeros (and a block entirely past S gets scale 0). The head's D features land in a prepared
// row of DK >= D (the kernel's head size), zero past D: zeros change neither a score nor a block's max.
template <int DT, bool SAGE>
__global__ __launch_bounds__(256) void attn_qk_prep_kernel(const void* __restrict__ src, int64_t S, int64_t Sp, int D, int DK,
                                                           int64_t stride, const float* __restrict__ mean,
                                                           int8_t* __restrict__ dst, float* __restrict__ scales) {
    __shared__ float red[4];
    const int64_t nbp = Sp / kAttnRows, b = blockIdx.x % nbp, h = blockIdx.x / nbp, r0 = b * kAttnRows;
    const int tid = threadIdx.x, n = kAttnRows * DK;
    const int64_t base = r0 * stride + h * D;
    if constexpr (SAGE) {
        float m = 0.0f;
        for (int e = tid; e < n; e += 256) {
            const int r = e / DK, d = e % DK;
            if (r0 + r < S && d < D) m = fmaxf(m, fabsf(attn_elem<DT>(src, base + r * stride + d) - (mean ? mean[h * D + d] : 0.0f)));
        }
        m = wave_max<64>(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        if (tid == 0) scales[h * nbp + b] = m / 127.0f;
        for (int e = tid; e < n; e += 256) {
            const int r = e / DK, d = e % DK;
            float c = 0.0f;
            if (r0 + r < S && d < D) {
                c = roundf((attn_elem<DT>(src, base + r * stride + d) - (mean ? mean[h * D + d] : 0.0f)) * inv);
                c = fminf(fmaxf(c, -127.0f), 127.0f);
            }
            dst[(h * Sp + r0 + r) * DK + d] = (int8_t) c;
        }
    } else {
        uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
        for (int e = tid; e < n; e += 256) {
            const int r = e / DK, d = e % DK;
            d16[(h * Sp + r0 + r) * DK + d] =
                r0 + r < S && d < D ? half_bits(attn_elem<DT>(src, base + r * stride + d)) : (uint16_t) 0;
        }
    }
}

// The same two preparations with 16-byte loads, for rows that are 16-byte aligned (the tensor and the stride): a
// thread holds its chunks (V values each) of the block's 64 rows in registers between the max and the codes.
template <int DT, bool SAGE, int D>
__global__ __launch_bounds__(256) void attn_qk_prep_vec_kernel(const void* __restrict__ src, int64_t S, int64_t Sp,
                                                               int64_t stride, const float* __restrict__ mean,
                                                               int8_t* __restrict__ dst, float* __restrict__ scales) {
    constexpr int V = Vec<DT>::V, CPR = D / V, N = kAttnRows * CPR / 256;   // chunks a row, chunks a thread
    __shared__ float red[4];
    const int64_t nbp = Sp / kAttnRows, b = blockIdx.x % nbp, h = blockIdx.x / nbp, r0 = b * kAttnRows;
    const int tid = threadIdx.x;
    const char* base = reinterpret_cast<const char*>(src) + (r0 * stride + h * D) * (int64_t) (16 / V);
    float v[N][V];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = tid + 256 * k, r = u / CPR, c = u % CPR;
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (r0 + r < S) raw = ld_nt(base + (int64_t) r * stride * (16 / V) + 16 * c);
        Vec<DT>::unpack(raw, v[k]);
    }
    if constexpr (SAGE) {
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int u = tid + 256 * k, r = u / CPR, c = u % CPR;
            if (mean) {
#pragma unroll
                for (int e = 0; e < V; ++e) v[k][e] = v[k][e] - mean[h * D + c * V + e];
            }
            if (r0 + r < S)
#pragma unroll
                for (int e = 0; e < V; ++e) m = fmaxf(m, fabsf(v[k][e]));
        }
        m = wave_max<64>(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        if (tid == 0) scales[h * nbp + b] = m / 127.0f;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int u = tid + 256 * k, r = u / CPR, c = u % CPR;
            uint32_t w[V / 4];
#pragma unroll
            for (int g = 0; g < V / 4; ++g) {
                float q[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float cc = roundf(v[k][4 * g + e] * inv);
                    cc = fminf(fmaxf(cc, -127.0f), 127.0f);
                    q[e] = r0 + r < S ? cc : 0.0f;
                }
                w[g] = (uint32_t) ((int) q[0] & 255) | ((uint32_t) ((int) q[1] & 255) << 8) |
                       ((uint32_t) ((int) q[2] & 255) << 16) | ((uint32_t) ((int) q[3] & 255) << 24);
            }
            int8_t* o = dst + (h * Sp + r0 + r) * D + c * V;
            if constexpr (V == 8) *reinterpret_cast<uint2*>(o) = make_uint2(w[0], w[1]);
            else *reinterpret_cast<uint32_t*>(o) = w[0];
        }
    } else {
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int u = tid + 256 * k, r = u / CPR, c = u % CPR;
            uint32_t w[V / 2];
#pragma unroll
            for (int g = 0; g < V / 2; ++g) w[g] = pack_f16(v[k][2 * g], v[k][2 * g + 1]);
            uint16_t* o = reinterpret_cast<uint16_t*>(dst) + (h * Sp + r0 + r) * D + c * V;
            if constexpr (V == 8) *reinterpret_cast<uint4*>(o) = make_uint4(w[0], w[1], w[2], w[3]);
            else *reinterpret_cast<uint2*>(o) = make_uint2(w[0], w[1]);
        }
    }
}

template <int DT, int D>
__global__ __launch_bounds__(256) void attn_v_prep_vec_kernel(const void* __restrict__ v, int64_t S, int64_t Sp,
                                                              int64_t stride, uint16_t* __restrict__ vt) {
    constexpr int V = Vec<DT>::V, CPR = D / V, N = kAttnRows * CPR / 256, PITCH = kAttnRows + 8;
    __shared__ uint16_t tile[D * PITCH];                     // [feature][token], half bits
    const int64_t nbp = Sp / kAttnRows, b = blockIdx.x % nbp, h = blockIdx.x / nbp, t0 = b * kAttnRows;
    const int tid = threadIdx.x;
    const char* base = reinterpret_cast<const char*>(v) + (t0 * stride + h * D) * (int64_t) (16 / V);
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = tid + 256 * k, t = u / CPR, c = u % CPR;
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (t0 + t < S) raw = ld_nt(base + (int64_t) t * stride * (16 / V) + 16 * c);
        float f[V];
        Vec<DT>::unpack(raw, f);
#pragma unroll
        for (int e = 0; e < V; ++e) tile[(c * V + e) * PITCH + t] = half_bits(f[e]);
    }
    __syncthreads();
    // output row d holds the 64 tokens: 8 chunks of 16 bytes
#pragma unroll
    for (int k = 0; k < D * 8 / 256; ++k) {
        const int u = tid + 256 * k, d = u / 8, c = u % 8;
        const uint4 val = *reinterpret_cast<const uint4*>(tile + d * PITCH + 8 * c);
        *reinterpret_cast<uint4*>(vt + (h * D + d) * Sp + t0 + 8 * c) = val;
    }
}

// v of one head and 64 tokens to half, transposed: vt [H, DK, Sp]; tokens past S and features past D become zeros
template <int DT>
__global__ __launch_bounds__(256) void attn_v_prep_kernel(const void* __restrict__ v, int64_t S, int64_t Sp, int D, int DK,
                                                          int64_t stride, uint16_t* __restrict__ vt) {
    __shared__ uint16_t tile[kAttnRows * (kAttnMaxD + 2)];
    const int64_t nbp = Sp / kAttnRows, b = blockIdx.x % nbp, h = blockIdx.x / nbp, t0 = b * kAttnRows;
    const int tid = threadIdx.x, n = kAttnRows * DK, pitch = DK + 2;
    for (int e = tid; e < n; e += 256) {
        const int t = e / DK, d = e % DK;
        tile[t * pitch + d] = t0 + t < S && d < D ? half_bits(attn_elem<DT>(v, (t0 + t) * stride + h * D + d)) : (uint16_t) 0;
    }
    __syncthreads();
    for (int e = tid; e < n; e += 256) {
        const int d = e / kAttnRows, t = e % kAttnRows;
        vt[(h * DK + d) * Sp + t0 + t] = tile[t * pitch + d];
    }
}

// ---- the attention kernel ----
struct AttnArgs {
    const int8_t* q;          // [H, Sp, D]: int8 codes (SAGE) or half bits
    const int8_t* k;
    const uint16_t* vt;       // [H, D, Sp] half bits
    const float* qs;          // [H, Sp / 64] (SAGE)
    const float* ks;
    int64_t S, Sp, H;
    float c;                  // log2(e) * fl(1 / sqrt(D)): scores in base 2
    void* out;                // [S, H * D]
    int out_dt;
    int D;                    // the heads' features (the kernel's DK of them are prepared, zero past D)
    int nqb;                  // blocks of 128 queries per head
    int kvdiv;                // query heads per key/value head: head h reads k and v of head h / kvdiv
    int64_t Spk;              // rows of the prepared k and v^T (Sp unless they come from another sequence)
};

// the chunk of row r (rows of CPR 16-byte chunks) where logical chunk c is stored: rows of fewer than 16 chunks
// change the pattern every 16 / CPR rows, longer rows every row
template <int CPR> __device__ __forceinline__ int attn_swz(int r, int c) {
    constexpr int RPS = CPR >= 16 ? 1 : 16 / CPR;
    return c ^ ((r / RPS) % CPR);
}

// {x of this lane, x of lane ^ 32} in some order
__device__ __forceinline__ float attn_pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float attn_pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// PAD: heads of D < DK features, or rows of out not on 16-byte boundaries: the output stores only features below D,
// four at a time where they stay aligned
template <bool SAGE, int DK, bool CAUSAL = false, bool PAD = false>
__global__ __launch_bounds__(256, DK == 256 ? 1 : 3) void attn_kernel(AttnArgs P) {
    constexpr int ESZ = SAGE ? 1 : 2, RB = DK * ESZ, CPR = RB / 16, NQF = RB / 32;
    constexpr int KTB = kAttnRows * RB, VTB = DK * kAttnRows * 2, STAGE = KTB + VTB;
    constexpr int NDT = DK / 32;                               // 32-row tiles of V^T (32 features each)
    __shared__ __attribute__((aligned(16))) int8_t lds[2 * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hl = lane >> 5, ql = lane & 31;
    const int64_t h = blockIdx.x / P.nqb, qb = blockIdx.x % P.nqb, Sp = P.Sp, S = P.S;
    const int64_t q0 = qb * kAttnQBlock + 32 * wave;          // this wavefront's first query
    const int64_t nbp = Sp / kAttnRows;
    // CAUSAL: query i sees keys 0 .. i, so the block stops at its last query
    const int64_t kend = CAUSAL ? (qb * kAttnQBlock + kAttnQBlock < S ? qb * kAttnQBlock + kAttnQBlock : S) : S;
    const int ntiles = (int) ((kend + kAttnRows - 1) / kAttnRows);

    // this lane's query fragments (second operand of the score products), held for the whole key walk
    v4i_a qf[NQF];
    {
        const int8_t* qrow = P.q + ((h * Sp + q0 + ql) * DK) * ESZ;
#pragma unroll
        for (int kk = 0; kk < NQF; ++kk) qf[kk] = *reinterpret_cast<const v4i_a*>(qrow + 32 * kk + 16 * hl);
    }
    const float fq = SAGE ? P.qs[h * nbp + q0 / kAttnRows] * P.c : P.c;

    // direct loads of key tile t into stage st: the K rows (64 x RB bytes) and the V^T rows (DK x 128 bytes)
    const int64_t g = h / P.kvdiv, Spk = P.Spk;              // the key/value head and its rows
    const int8_t* kbase = P.k + g * Spk * RB;
    const uint16_t* vbase = P.vt + g * DK * Spk;
    auto issue = [&](int t, int st) {
        int8_t* s = lds + st * STAGE;
        constexpr int KI = CPR / 4;                            // K instructions a wavefront
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int i = wave * KI + j, u = 64 * i + lane, r = u / CPR, c = attn_swz<CPR>(r, u % CPR);
            const int8_t* gk = kbase + ((int64_t) t * kAttnRows + r) * RB + 16 * c;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*) gk,
                                             (__attribute__((address_space(3))) void*) (s + 1024 * i), 16, 0, 0);
        }
        constexpr int VI = DK / 32;                              // V^T instructions a wavefront (DK * 8 units / 64 / 4)
#pragma unroll
        for (int j = 0; j < VI; ++j) {
            const int i = wave * VI + j, u = 64 * i + lane, r = u / 8, c = attn_swz<8>(r, u % 8);
            const uint16_t* gv = vbase + (int64_t) r * Spk + (int64_t) t * kAttnRows + 8 * c;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*) gv,
                                             (__attribute__((address_space(3))) void*) (s + KTB + 1024 * i), 16, 0, 0);
        }
    };

    v16f_a o[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) o[i] = (v16f_a) 0.0f;
    float m = -INFINITY, l = 0.0f;

    // one 64-key tile; TAIL: the last tile, which holds keys past S
    auto step = [&](int t, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        wait_vm<0>();
        __syncthreads();                                       // tile t is in; every wavefront is done with tile t - 1
        if (t + 1 < ntiles) issue(t + 1, (t + 1) & 1);
        const int8_t* st = lds + (t & 1) * STAGE;

        // ---- scores: two 32-key halves of the tile ----
        float x[32];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = 32 * j + ql;
            // the half's NQF fragments of K read together, then its NQF products
            v4i_a kf[NQF];
#pragma unroll
            for (int kk = 0; kk < NQF; ++kk) kf[kk] = *reinterpret_cast<const v4i_a*>(st + (r * CPR + attn_swz<CPR>(r, 2 * kk + hl)) * 16);
            if constexpr (SAGE) {
                v16i_a a = (v16i_a) 0;
#pragma unroll
                for (int kk = 0; kk < NQF; ++kk) a = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[kk], qf[kk], a, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; ++i) x[16 * j + i] = (float) a[i];
            } else {
                v16f_a a = (v16f_a) 0.0f;
#pragma unroll
                for (int kk = 0; kk < NQF; ++kk)
                    a = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_a, kf[kk]), __builtin_bit_cast(v8h_a, qf[kk]), a, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; ++i) x[16 * j + i] = a[i];
            }
        }
        // register i of half j holds key 32 j + 8 (i / 4) + 4 hl + i % 4 of the tile. The scale f > 0 is applied after
        // the max (max(a f) = f max(a)) and inside the exponent: p = 2^(a f - m) with one fused multiply-add.
        const float f = SAGE ? fq * P.ks[g * nbp + t] : fq;
        // register i holds key 64 t + 4 hl + off(i); it is live below S and, CAUSAL, up to this lane's query
        int lim = (int) (S - (int64_t) t * kAttnRows) - 4 * hl;
        if constexpr (CAUSAL) {
            const int qlim = (int) (q0 + ql - (int64_t) t * kAttnRows) - 4 * hl + 1;
            lim = lim < qlim ? lim : qlim;
        }
        auto live = [&](int i) { return 32 * (i / 16) + 8 * ((i % 16) / 4) + i % 4 < lim; };
        if constexpr (TAIL) {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (!live(i)) x[i] = -INFINITY;
        }
        float mx = x[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) mx = fmaxf(mx, x[i]);
        mx = attn_pair_max(mx) * f;
        // The reference point m of the exponents moves only when some lane's tile max passes it by more than 8 (in
        // base 2): the weights then stay at most 2^8, exact in half's range, and O / l does not depend on m. O and l
        // are rescaled only then (the empty asm keeps the compiler from running the 64 multiplies unconditionally).
        if (__any(mx > m + 8.0f)) {
            asm volatile("" ::: "memory");
            const float mn = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
            l = l * alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) o[dt] = o[dt] * alpha;
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], f, -m));
        if constexpr (TAIL) {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (!live(i)) x[i] = 0.0f;
        }
        float ls = 0.0f;

        // ---- O^T += V^T P^T, 16 keys a product ----
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // keys 16 s + 4 hl + (0..3) and 16 s + 8 + 4 hl + (0..3) of this lane's query, as half pairs
            const int b = 16 * (s / 2) + 8 * (s % 2);
            uint32_t a0 = pack_f16(x[b + 0], x[b + 1]), a1 = pack_f16(x[b + 2], x[b + 3]);
            uint32_t b0 = pack_f16(x[b + 4], x[b + 5]), b1 = pack_f16(x[b + 6], x[b + 7]);
            // the row sum of the weights as rounded to half (the ones P v uses), two at a time
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, a0), h2_one, ls, false);
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, a1), h2_one, ls, false);
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, b0), h2_one, ls, false);
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, b1), h2_one, ls, false);
            // the upper half's first group for the lower half's second: each lane then has keys 16 s + 8 hl + (0..7)
            const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
            a0 = s0[0]; b0 = s0[1]; a1 = s1[0]; b1 = s1[1];
            v4i_a pf;
            pf[0] = (int) a0; pf[1] = (int) a1; pf[2] = (int) b0; pf[3] = (int) b1;
            const v8h_a pb = __builtin_bit_cast(v8h_a, pf);
            // the step's NDT fragments of V^T read together, then its NDT products
            v4i_a vf[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const int r = 32 * dt + ql;
                vf[dt] = *reinterpret_cast<const v4i_a*>(st + KTB + (r * 8 + attn_swz<8>(r, 2 * s + hl)) * 16);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_a, vf[dt]), pb, o[dt], 0, 0, 0);
        }
        l = l + ls;
    };
    issue(0, 0);
    // tiles with no key past S (and, CAUSAL, none past the block's first query) need no mask
    int full = (int) (S / kAttnRows);
    if constexpr (CAUSAL) full = full < (int) (qb * kAttnQBlock / kAttnRows) ? full : (int) (qb * kAttnQBlock / kAttnRows);
    for (int t = 0; t < full; ++t) step(t, std::false_type{});
    for (int t = full; t < ntiles; ++t) step(t, std::true_type{});

    // ---- out = O / l, rounded to half, in out's type: the head's D features (of the DK computed) ----
    const float inv = 1.0f / attn_pair_sum(l);
    const int64_t qi = q0 + ql;
    if (qi < S) {
        const int esz = P.out_dt == H3S_F32 ? 4 : 2, D = PAD ? P.D : DK;
        char* orow = reinterpret_cast<char*>(P.out) + ((qi * P.H + h) * D) * esz;
        // four features a store when D keeps every group of four on a 4-element boundary, else one at a time
        const bool quads = !PAD || (D % 4 == 0 && (reinterpret_cast<uintptr_t>(P.out) & 15) == 0);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                // registers 4 g .. 4 g + 3 of o[dt]: features 32 dt + 8 g + 4 hl + (0..3)
                const int f0 = 32 * dt + 8 * g + 4 * hl;
                if (PAD && f0 >= D) continue;
                float v[4];
#pragma unroll
                // the reference's result buffer is half for the two forms of h3s_attention; its causal kernel stores
                // acc / l straight into out's type
                for (int i = 0; i < 4; ++i) v[i] = CAUSAL ? o[dt][4 * g + i] * inv : round_f16(o[dt][4 * g + i] * inv);
                char* at = orow + f0 * esz;
                if (quads) {
                    if (P.out_dt == H3S_F32) *reinterpret_cast<float4*>(at) = make_float4(v[0], v[1], v[2], v[3]);
                    else if (P.out_dt == H3S_BF16) *reinterpret_cast<uint2*>(at) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
                    else *reinterpret_cast<uint2*>(at) = make_uint2(pack_f16(v[0], v[1]), pack_f16(v[2], v[3]));
                } else if constexpr (PAD) {
                    for (int i = 0; i < 4 && f0 + i < D; ++i) {
                        if (P.out_dt == H3S_F32) reinterpret_cast<float*>(at)[i] = v[i];
                        else if (P.out_dt == H3S_BF16) reinterpret_cast<uint16_t*>(at)[i] = (uint16_t) pack_bf16(v[i], 0.0f);
                        else reinterpret_cast<uint16_t*>(at)[i] = (uint16_t) pack_f16(v[i], 0.0f);
                    }
                }
            }
    }
}

}  // namespace h3
