// attn_impl.h - attention on gfx950's matrix cores: out = softmax(q k^T / sqrt(D)) v per head (kernels/h3sycl.h:185-192),
// in the reference's two forms (kernels/h3sycl.cpp:1676-1767 and 1496-1550):
//   SAGE:  q and k - mean(k) as int8 with one scale per head per 64 rows (the preparation kernels below restate the
//          reference's quantization exactly), scores on the i8 matrix cores, exact in int32;
//   16-bit: q and k in IEEE half, scores on the f16 matrix cores with float32 accumulation.
// Both: v in IEEE half, the softmax online in float32 (base 2), P in half, P v on the f16 matrix cores, the result
// divided by the row sum, rounded to half (the reference's result buffer is half) and stored in out's type.
//
// Layouts (prepared once per call, in the context's scratch): codes or halves of q and k [H, Sp, DK], v transposed to
// half [H, DK, Sp] (keys permuted inside each group of 16: attn_vt_pos), Sp = S rounded up to 128 (256 for the
// pipelined kernel) with zero rows, DK = the head size D rounded up to 64, 128 or 256 with zero
// features (which change no score and no block max); the output keeps the D features. One block = 4 wavefronts = 128 queries of one head; a
// wavefront owns 32 queries and walks all keys 64 at a time. Per 64-key tile:
//   S^T = K Q^T:  v_mfma_i32_32x32x32_i8 (or f32_32x32x16_f16) with K as the first operand, so every lane ends with
//                 scores of one query (lane % 32) for 32 of the 64 keys (the other 32 in lane ^ 32);
//   softmax:      the row max needs one exchange with lane ^ 32 (v_permlane32_swap); the exponents' reference
//                 point moves only when a tile max passes it by 2^8; the row sum stays a per-lane partial until the end;
//   O^T += V^T P^T: v_mfma_f32_32x32x16_f16 with V^T as the first operand; P's registers are the second operand as
//                 they are, since v^T stores each 16-key group's keys in the order the score registers hold them.
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

// One direct global -> LDS load (16 bytes a lane to lds + 16 lane) written as inline asm: the compiler then does
// not track it, where for the builtin it makes every later LDS read wait for all direct loads in flight (it cannot
// tell the stages apart), which would make a ring's reads of a landed stage wait for the refills issued after it. The
// caller's wait_vm before each barrier orders these loads; the memory clobber keeps the compiler from moving LDS
// accesses across them.
// (m0 is the compiler's reserved register: it holds nothing across these statements)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void attn_dma16(const void* g, const void* lds_dst) {
    const uint32_t m = (uint32_t) (uintptr_t) lds_dst;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}
#pragma clang diagnostic pop

// k's mean over the sequence per (head, feature): a float32 sum in token order, / S (h3sycl.cpp:1732-1737). Each
// feature's sum is one serial chain of S additions (a wavefront issues a dependent v_add_f32 every 4.9 cycles), and
// the features are few (4096 at 32 heads of 128), so the kernel spreads them thin to use every CU's memory
// parallelism: a block takes F features (16: 256 blocks at 4096 features; a block's loads in flight, not HBM, bound
// the rate; 32 where 16 would make more blocks than CUs, so that the serial chains run in one round: 224 blocks at
// the DiT's 56 heads of 128), one a lane of wavefront 0, which only reads four float32 rows of its feature at a time
// (ds_read_b128) and adds them in order. Wavefronts 1-3 keep seven row chunks in flight with direct loads (attn_dma16) into a ring of
// eight 12 KiB stages (row-major, as in memory) and turn each landed chunk into float32 rows per feature
// (feature-major, padded) in one of two buffers. One barrier a chunk: after barrier i, wavefront 0 sums chunk i - 1
// while the others convert chunk i, refill chunk i - 1's stage with chunk i + 7 and wait for chunk i + 1. A chunk
// past the last loads the last one again (into a stage no chunk uses then), so the wait is the same at every chunk.
// Blocks of neighbouring features (which share 128-byte lines) are numbered onto one XCD. Needs the rows 16-byte
// aligned (k and the stride); attn_kmean_rows_kernel is the general form.
constexpr int kKmeanFeat = 16, kKmeanFeatWide = 32, kKmeanStages = 8, kKmeanChunk = 12288, kKmeanLoaders = 192;
template <int DT, int F>
__global__ __launch_bounds__(256) void attn_kmean_kernel(const void* __restrict__ k, int64_t S, int64_t stride,
                                                         float* __restrict__ mean) {
    constexpr int ESZ = DT == H3S_F32 ? 4 : 2, RB = F * ESZ;   // bytes of a row's F features
    constexpr int SEG = RB / 16, ROWS = kKmeanChunk / RB, LPT = kKmeanChunk / (kKmeanLoaders * 16);
    constexpr int VS = 16 / ESZ;                 // values of a 16-byte segment
    constexpr int TS = ROWS + 4;                 // floats a feature takes in a converted buffer
    constexpr int SUB = 32;                      // rows a sub-batch of the sums (8 reads in flight)
    static_assert(kKmeanChunk % RB == 0 && kKmeanChunk % (kKmeanLoaders * 16) == 0, "attn_kmean_kernel: chunk shape");
    static_assert(kKmeanLoaders % SEG == 0 && kKmeanLoaders / SEG * 4 == ROWS && ROWS % SUB == 0,
                  "attn_kmean_kernel: a loader converts 4 rows of a segment");
    __shared__ __attribute__((aligned(16))) uint8_t ring[kKmeanStages * kKmeanChunk];
    __shared__ __attribute__((aligned(16))) float conv[2][F * TS];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blocks go to the 8 XCDs round robin: renumbered so that each XCD takes a contiguous run of features
    int64_t b = blockIdx.x;
    if (gridDim.x % 8 == 0) b = (b % 8) * (gridDim.x / 8) + b / 8;
    const int64_t c0 = b * F, nch = (S + ROWS - 1) / ROWS;
    const char* base = reinterpret_cast<const char*>(k) + c0 * ESZ;
    // loader thread p = tid - 64, load j: unit u = p + 192 j of the chunk (row u / SEG, 16-byte segment u % SEG),
    // landing at byte 16 u of the stage (1024 (3 j + wave - 1) + 16 lane): the stage is the chunk row-major
    auto issue = [&](int64_t ch) {
        const int64_t cc = ch < nch ? ch : nch - 1;
        uint8_t* st = ring + (ch % kKmeanStages) * kKmeanChunk;
#pragma unroll
        for (int j = 0; j < LPT; ++j) {
            const int u = (tid - 64) + kKmeanLoaders * j;
            int64_t row = cc * ROWS + u / SEG;
            row = row < S ? row : S - 1;
            attn_dma16(base + row * stride * ESZ + 16 * (u % SEG), st + (3 * j + wave - 1) * 1024);
        }
    };
    // loader thread p converts rows 4 g .. 4 g + 3 of segment s (g = p / SEG, s = p % SEG): four 16-byte reads, then
    // four rows of each of the segment's VS features as one 16-byte write
    auto convert = [&](int64_t ch) {
        const int p = tid - 64, sg = p % SEG, g = p / SEG;
        const uint8_t* st = ring + (ch % kKmeanStages) * kKmeanChunk;
        float* cv = conv[ch & 1];
        uint4 raw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) raw[r] = *reinterpret_cast<const uint4*>(st + (4 * g + r) * RB + 16 * sg);
        float x[4][VS];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t w[4] = {raw[r].x, raw[r].y, raw[r].z, raw[r].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (DT == H3S_F32) x[r][i] = __uint_as_float(w[i]);
                else if constexpr (DT == H3S_BF16) { x[r][2 * i] = bf16_lo(w[i]); x[r][2 * i + 1] = bf16_hi(w[i]); }
                else { x[r][2 * i] = f16_lo(w[i]); x[r][2 * i + 1] = f16_hi(w[i]); }
            }
        }
#pragma unroll
        for (int e = 0; e < VS; ++e)
            *reinterpret_cast<float4*>(cv + (VS * sg + e) * TS + 4 * g) = make_float4(x[0][e], x[1][e], x[2][e], x[3][e]);
    };
    float sum = 0.0f;
    if (wave > 0) {
        for (int64_t ch = 0; ch < kKmeanStages - 1; ++ch) issue(ch);
        wait_vm<(kKmeanStages - 2) * LPT>();     // chunk 0 has landed
    }
    lds_barrier();
    for (int64_t i = 0; i <= nch; ++i) {
        if (wave == 0) {
            if (i >= 1 && lane < F) {
                const float* cf = conv[(i - 1) & 1] + lane * TS;
                const int rows = S - (i - 1) * ROWS < ROWS ? (int) (S - (i - 1) * ROWS) : ROWS;
                if (rows == ROWS) {
                    // sub-batches of SUB rows, the next one's reads in flight during this one's additions
                    float4 f[2][SUB / 4];
#pragma unroll
                    for (int r = 0; r < SUB / 4; ++r) f[0][r] = *reinterpret_cast<const float4*>(cf + 4 * r);
#pragma unroll
                    for (int sb = 0; sb < ROWS / SUB; ++sb) {
                        if (sb + 1 < ROWS / SUB)
#pragma unroll
                            for (int r = 0; r < SUB / 4; ++r)
                                f[(sb + 1) & 1][r] = *reinterpret_cast<const float4*>(cf + (sb + 1) * SUB + 4 * r);
#pragma unroll
                        for (int r = 0; r < SUB / 4; ++r) {
                            sum = sum + f[sb & 1][r].x;
                            sum = sum + f[sb & 1][r].y;
                            sum = sum + f[sb & 1][r].z;
                            sum = sum + f[sb & 1][r].w;
                        }
                    }
                } else {
                    for (int r = 0; r < rows; ++r) sum = sum + cf[r];
                }
            }
        } else if (i < nch) {
            convert(i);
            issue(i + kKmeanStages - 1);         // into chunk i - 1's stage, converted before the last barrier
            wait_vm<(kKmeanStages - 2) * LPT>(); // chunk i + 1 has landed
        }
        lds_barrier();                           // chunk i converted, chunk i + 1 in, chunk i - 1's sums read
    }
    if (wave > 0) wait_vm<0>();                  // no direct load outlives the block
    else if (lane < F) mean[c0 + lane] = sum / (float) S;
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
// Where key t of a 64-key tile sits in its row of v^T: inside each group of 16 keys the middle two quads swap
// (bits 2 and 3 of t). The score products leave key 16 s + 8 (j / 4) + 4 hl + j % 4 of a query in register 8 s + j
// of lane half hl; the P v product's second operand takes 8 consecutive k-indices per lane half from the registers
// as they are, so its first operand (a 16-byte chunk of a v^T row) must hold those same 8 keys, in that order.
__host__ __device__ constexpr int attn_vt_pos(int t) { return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1); }

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
    // k's mean at this thread's chunks, loaded before the rows so that both are in flight together (loaded after
    // them, each chunk's mean waited for the rows and then for itself)
    float mk[N][V];
    if constexpr (SAGE) {
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int c = (tid + 256 * k) % CPR;
#pragma unroll
            for (int e = 0; e < V; e += 4) {
                const float4 t = mean ? *reinterpret_cast<const float4*>(mean + h * D + c * V + e) : make_float4(0.f, 0.f, 0.f, 0.f);
                mk[k][e] = t.x; mk[k][e + 1] = t.y; mk[k][e + 2] = t.z; mk[k][e + 3] = t.w;
            }
        }
    }
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
            const int u = tid + 256 * k, r = u / CPR;
            if (mean) {
#pragma unroll
                for (int e = 0; e < V; ++e) v[k][e] = v[k][e] - mk[k][e];
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
    // PITCH: an odd number of 4-byte words a feature row (35), so the 16 chunks a wavefront's lanes write for one
    // token group fall in distinct banks (a pitch of 36 words put 8 lanes on each bank: 29.9 -> 21.4 us on average
    // over the attention calls of a benchmark run); the rows are then 4-byte aligned, read 4 bytes at a time
    constexpr int V = Vec<DT>::V, CPR = D / V, N = kAttnRows * CPR / 256, PITCH = kAttnRows + 6;
    __shared__ __attribute__((aligned(16))) uint16_t tile[D * PITCH];   // [feature][token], half bits
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
    // output row d holds the 64 tokens in the key order attn_vt_pos sets: chunk 2 g + e (8 tokens) is tokens
    // 16 g + 4 e + (0..3) then 16 g + 8 + 4 e + (0..3)
#pragma unroll
    for (int k = 0; k < D * 8 / 256; ++k) {
        const int u = tid + 256 * k, d = u / 8, c = u % 8, t = 16 * (c / 2) + 4 * (c % 2);
        const uint32_t* row = reinterpret_cast<const uint32_t*>(tile + d * PITCH + t);
        *reinterpret_cast<uint4*>(vt + (h * D + d) * Sp + t0 + 8 * c) = make_uint4(row[0], row[1], row[4], row[5]);
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
        vt[(h * DK + d) * Sp + t0 + attn_vt_pos(t)] = tile[t * pitch + d];
    }
}

// two floats to a pair of halves (round to nearest even), left for the compiler to place: the exponentials can then
// be written straight into the register pair v_cvt_pk_f16_f32 reads
__device__ __forceinline__ uint32_t attn_pack_h2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2_a));
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
    int nqb;                  // query blocks per head (of 128 queries, or 256 in the pipelined kernel)
    int kvdiv;                // query heads per key/value head: head h reads k and v of head h / kvdiv
    int64_t Spk;              // rows of the prepared k and v^T (Sp unless they come from another sequence)
    // the pipelined kernel's split of the last round: blocks [nfull, nfull + tail * nsplit) each take key tiles
    // [s ts, s ts + ts) of query block nfull + (b - nfull) / nsplit (s = (b - nfull) % nsplit) and leave O, m and l
    // in po / pml for attn_merge_kernel; nfull = the grid and nsplit = 1 when nothing is split
    int64_t nfull;
    int nsplit, ts;
    float* po;                // [tail * nsplit, 256, DK] O before the division by l
    float* pml;               // [tail * nsplit, 256, 2] m and l
    // the pipelined kernel with qraw set reads q from the caller's rows (stride qstride elements of type q_dt, 16-byte
    // aligned) and forms its fragments itself, as attn_qk_prep_vec_kernel would (q and qs are then unused)
    const void* qraw;
    int64_t qstride;
    int q_dt;
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
    float ks_cur = SAGE ? P.ks[g * nbp] : 0.0f;               // SAGE: k's scale of the tile being computed

    // one 64-key tile; TAIL: the last tile, which holds keys past S
    auto step = [&](int t, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        wait_vm<0>();
        __syncthreads();                                       // tile t is in; every wavefront is done with tile t - 1
        // SAGE: the next tile's k scale, loaded before the tile's direct loads and waited for with them at the next
        // step (loaded after them, its wait here would wait for the whole tile)
        const float ks_next = SAGE ? P.ks[g * nbp + (t + 1 < ntiles ? t + 1 : t)] : 0.0f;
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
        const float f = SAGE ? fq * ks_cur : fq;
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
            const uint32_t a0 = attn_pack_h2(x[b + 0], x[b + 1]), a1 = attn_pack_h2(x[b + 2], x[b + 3]);
            const uint32_t b0 = attn_pack_h2(x[b + 4], x[b + 5]), b1 = attn_pack_h2(x[b + 6], x[b + 7]);
            // the row sum of the weights as rounded to half (the ones P v uses), two at a time
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, a0), h2_one, ls, false);
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, a1), h2_one, ls, false);
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, b0), h2_one, ls, false);
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, b1), h2_one, ls, false);
            // as they are: v^T's keys are stored in this order (attn_vt_pos)
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
        ks_cur = ks_next;
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



constexpr int kAttnPPQ = 256;            // queries of a pipelined block
// 1.5 2^23: for |n| < 2^22 the float kScoreBias + n has the bits kScoreBiasBits + n, so int32 score products started
// from kScoreBiasBits read as floats without a conversion; |score| <= 128 127^2 < 2^22 for heads of 128 features
constexpr float kScoreBias = 12582912.0f;
constexpr int kScoreBiasBits = 0x4B400000;
constexpr int kAttnPPTiles = 4096;       // key tiles it takes (sequences of up to 262144 tokens)


// ---- the pipelined form: heads of 128 features, no mask but the sequence's end (both forms) ----
// One block = 8 wavefronts = 256 queries of one head, 32 a wavefront as above, two wavefronts a SIMD. Each step a
// wavefront computes the scores of key tile t + 1, then tile t's P v products with the softmax of tile t + 1 (the
// two are independent) between them: a wavefront issues a few VALU instructions between its own matrix products at
// no cost to them, and both wavefronts of a SIMD do so. One workgroup barrier a step.
// Key tile j is read in steps j - 1 (its K) and j (its V^T); a ring of NS stages holds it; its stage is refilled
// (tile j + NS) at the start of step j + 1, every wavefront issuing its share of the direct loads, which it waits for
// before the barrier that publishes them. The ring's loads are inline asm (attn_dma16), the head's k scales are
// copied into LDS once, and the int8 score products start from kScoreBias's bits: see the helpers above.
// A block of a split last round (AttnArgs::nfull) walks only its range of key tiles, counted from its first, and
// leaves O, m and l to attn_merge_kernel.
template <bool SAGE, int NS>
__global__ __launch_bounds__(512, 1) void attn_pl_kernel(AttnArgs P) {
    constexpr int DK = 128, ESZ = SAGE ? 1 : 2, RB = DK * ESZ, CPR = RB / 16, NQF = RB / 32;
    constexpr int KTB = kAttnRows * RB, VTB = DK * kAttnRows * 2, STAGE = KTB + VTB;
    constexpr int NDT = DK / 32;
    constexpr int KI = KTB / 1024 / 8, VI = VTB / 1024 / 8;   // direct loads of a wavefront a tile (K, V^T)
    constexpr int LATER = (NS - 3) * (KI + VI);                // loads of later tiles in flight at a tile's wait
    static_assert(NS >= 3 && KI >= 1 && VI >= 1, "ring");
    __shared__ __attribute__((aligned(16))) int8_t lds[NS * STAGE];
    // SAGE: the key tiles' scales of the head, copied once (a global load in the loop would sit behind the ring's
    // direct loads in the same wait counter)
    __shared__ float ksl[SAGE ? kAttnPPTiles : 1];
    const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, ql = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blocks go to the 8 XCDs round robin: renumbered so that each XCD takes a contiguous run (the blocks of few
    // heads at a time, which then share K and V^T in its L2)
    // (32-bit block arithmetic: the host keeps the grid below 2^31; 64-bit divisions here delayed every block's start)
    int b = (int) blockIdx.x;
    // a block of the split last round: its query block and its range of key tiles (slot: its partial sums)
    int slot = -1, t0 = 0;
    const int nfull = (int) P.nfull, Tall = (int) ((P.S + kAttnRows - 1) / kAttnRows);
    int T = Tall;
    if (b < nfull) {
        if (nfull % 8 == 0) b = (b % 8) * (nfull / 8) + b / 8;
    } else {
        slot = b - nfull;
        b = nfull + slot / P.nsplit;
        t0 = (slot % P.nsplit) * P.ts;
        T = Tall - t0 < P.ts ? Tall - t0 : P.ts;
    }
    const int64_t h = b / P.nqb, qb = b % P.nqb, Sp = P.Sp, S = P.S;
    const int64_t q0 = qb * kAttnPPQ + 32 * wave;             // this wavefront's first query
    const int64_t nbp = Sp / kAttnRows;

    v4i_a qf[NQF];
    float fq = P.c;
    // With P.qraw: this lane's 64 features of its query straight from the caller's rows (fragment kk: FR features from
    // 32 kk + 16 hl for int8 codes, 16 kk + 8 hl for halves), turned into the fragments attn_qk_prep_vec_kernel would
    // have written: halves here; int8 codes after the prologue's barrier, where the two wavefronts of a 64-row scale
    // block (wavefronts 2j, 2j + 1) have each left their 32 rows' max in qmax. Rows past S are zeros.
    constexpr int FR = SAGE ? 16 : 8;
    __shared__ float qmax[8];
    float qx[NQF * FR];
    float qm = 0.0f;
    if (P.qraw) {
        const int64_t qi = q0 + ql;
        const int qes = P.q_dt == H3S_F32 ? 4 : 2;
        const char* qrow = reinterpret_cast<const char*>(P.qraw) + (qi * P.qstride + h * DK) * qes;
#pragma unroll
        for (int kk = 0; kk < NQF; ++kk) {
            const int f0 = SAGE ? 32 * kk + 16 * hl : 16 * kk + 8 * hl;
#pragma unroll
            for (int c8 = 0; c8 < FR; c8 += 8) {
                float* x = qx + kk * FR + c8;
                if (qi >= S) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
                } else if (P.q_dt == H3S_F32) {
                    const float4 a = *reinterpret_cast<const float4*>(qrow + (f0 + c8) * 4);
                    const float4 b = *reinterpret_cast<const float4*>(qrow + (f0 + c8) * 4 + 16);
                    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
                } else {
                    const uint4 u = *reinterpret_cast<const uint4*>(qrow + (f0 + c8) * 2);
                    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        x[2 * i] = P.q_dt == H3S_BF16 ? bf16_lo(w[i]) : f16_lo(w[i]);
                        x[2 * i + 1] = P.q_dt == H3S_BF16 ? bf16_hi(w[i]) : f16_hi(w[i]);
                    }
                }
            }
        }
        if constexpr (SAGE) {
#pragma unroll
            for (int i = 0; i < NQF * FR; ++i) qm = fmaxf(qm, fabsf(qx[i]));
            qm = wave_max<64>(qm);
            if (lane == 0) qmax[wave] = qm;
        } else {
#pragma unroll
            for (int kk = 0; kk < NQF; ++kk) {
                v4i_a w;
#pragma unroll
                for (int i = 0; i < 4; ++i) w[i] = (int) pack_f16(qx[kk * FR + 2 * i], qx[kk * FR + 2 * i + 1]);
                qf[kk] = w;
            }
        }
    } else {
        const int8_t* qrow = P.q + ((h * Sp + q0 + ql) * DK) * ESZ;
#pragma unroll
        for (int kk = 0; kk < NQF; ++kk) qf[kk] = *reinterpret_cast<const v4i_a*>(qrow + 32 * kk + 16 * hl);
        if constexpr (SAGE) fq = P.qs[h * nbp + q0 / kAttnRows] * P.c;
    }

    const int64_t g = h / P.kvdiv, Spk = P.Spk;
    if constexpr (SAGE)
        for (int i = tid; i < T; i += 512) ksl[i] = P.ks[g * nbp + t0 + i];
    // tiles are counted from t0 (this block's first key tile) from here on
    const int8_t* kbase = P.k + (g * Spk + (int64_t) t0 * kAttnRows) * RB;
    const uint16_t* vbase = P.vt + g * DK * Spk + (int64_t) t0 * kAttnRows;
    // tile t into stage t % NS; a tile past the last loads the last one again (into a stage no tile uses then), so
    // that every wavefront has the same loads in flight at every wait
    auto issue = [&](int t) {
        const int64_t tc = t < T ? t : T - 1;
        int8_t* s = lds + (t % NS) * STAGE;
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int i = wave * KI + j, u = 64 * i + lane, r = u / CPR, c = attn_swz<CPR>(r, u % CPR);
            const int8_t* gk = kbase + (tc * kAttnRows + r) * RB + 16 * c;
            attn_dma16(gk, s + 1024 * i);
        }
#pragma unroll
        for (int j = 0; j < VI; ++j) {
            const int i = wave * VI + j, u = 64 * i + lane, r = u / 8, c = attn_swz<8>(r, u % 8);
            const uint16_t* gv = vbase + (int64_t) r * Spk + tc * kAttnRows + 8 * c;
            attn_dma16(gv, s + KTB + 1024 * i);
        }
    };

    v16f_a o[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) o[i] = (v16f_a) 0.0f;
    float m = -INFINITY, l = 0.0f;
    typedef typename std::conditional<SAGE, v16i_a, v16f_a>::type score_t;
    score_t sc[2];                                             // the scores of the next tile, two 32-key halves
    v8h_a pb[4];                                               // the weights of the tile whose P v products run now
    v8h_a pn[4];                                               // the weights being formed for the next tile

    // the scores of tile t + 1 (K of its stage), two 32-key halves, started from kScoreBias's bits (SAGE)
    auto scores = [&](int t) {
        const int8_t* sk = lds + ((t + 1) % NS) * STAGE;
        sc[0] = sc[1] = SAGE ? (score_t) kScoreBiasBits : (score_t) 0;
        v4i_a kf[2][2];
        auto kread = [&](int u, v4i_a (&d)[2]) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = 32 * j + ql;
                d[j] = *reinterpret_cast<const v4i_a*>(sk + (r * CPR + attn_swz<CPR>(r, 2 * u + hl)) * 16);
            }
        };
        kread(0, kf[0]);
#pragma unroll
        for (int u = 0; u < NQF; ++u) {
            // the next sub-step's two K fragments read ahead of this one's products, fenced (the scheduler sinks
            // each read to its product otherwise, and its latency comes before the product)
            if (u + 1 < NQF) kread(u + 1, kf[(u + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if constexpr (SAGE) sc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[u & 1][j], qf[u], sc[j], 0, 0, 0);
                else sc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_a, kf[u & 1][j]),
                                                                     __builtin_bit_cast(v8h_a, qf[u]), sc[j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // O += P_t v_t: 16 products (V^T of tile t's stage)
    auto pv = [&](int t) {
        const int8_t* sv = lds + (t % NS) * STAGE + KTB;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            v4i_a vf[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const int r = 32 * dt + ql;
                vf[dt] = *reinterpret_cast<const v4i_a*>(sv + (r * 8 + attn_swz<8>(r, 2 * u + hl)) * 16);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h_a, vf[dt]), pb[u], o[dt], 0, 0, 0);
        }
    };
    // the softmax of the scores of tile t + 1 -> its half weights (pn), the running max and row sum; sets alpha when
    // O is to be rescaled (after this step's P v products, which use the old reference)
    auto softmax = [&](int t, auto tail_tag, float& alpha) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        const int tn = t + 1;
        // register i holds key 64 tn + 32 (i / 16) + 8 ((i % 16) / 4) + 4 hl + i % 4. SAGE: its bits are those of
        // the float kScoreBias + score (the score products start from kScoreBias's bits), read as they are.
        float x[32];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // the whole vector reinterpreted (an element-wise __builtin_bit_cast(float, sc[j][i]) compiled to copies
            // of element 0 here)
            const v16f_a xf = SAGE ? __builtin_bit_cast(v16f_a, sc[j]) : __builtin_convertvector(sc[j], v16f_a);
#pragma unroll
            for (int i = 0; i < 16; ++i) x[16 * j + i] = xf[i];
        }
        const float f = SAGE ? fq * ksl[tn] : fq;
        const int lim = (int) (S - (int64_t) (t0 + tn) * kAttnRows) - 4 * hl;
        auto live = [&](int i) { return 32 * (i / 16) + 8 * ((i % 16) / 4) + i % 4 < lim; };
        // The weights p = 2^(score f - m) rounded to half, packed into pb as the P v products take them, and their
        // sum over this lane's keys. SAGE: score f - m = x f - (kScoreBias f + m), with one rounding of the offset
        // (relative 2^-24 of kScoreBias f, far below half's rounding of p).
        // chunk s: the weights of registers 8 s .. 8 s + 7 into pn[s], their sum
        auto chunk = [&](int s, float c) {
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[8 * s + e], f, -c));
                    if (TAIL && !live(8 * s + e)) p[e] = 0.0f;
                }
                const uint32_t a0 = attn_pack_h2(p[0], p[1]), a1 = attn_pack_h2(p[2], p[3]);
                const uint32_t b0 = attn_pack_h2(p[4], p[5]), b1 = attn_pack_h2(p[6], p[7]);
                float ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, a0), h2_one, 0.0f, false);
                ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, a1), h2_one, ls, false);
                ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, b0), h2_one, ls, false);
                ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_a, b1), h2_one, ls, false);
                v4i_a pf;                                      // as they are (attn_vt_pos)
                pf[0] = (int) a0; pf[1] = (int) a1; pf[2] = (int) b0; pf[3] = (int) b1;
                pn[s] = __builtin_bit_cast(v8h_a, pf);
                return ls;
        };
        auto weights = [&]() {
            const float c = SAGE ? __builtin_fmaf(kScoreBias, f, m) : m;
            float ls[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) ls[s] = chunk(s, c);
            return (ls[0] + ls[1]) + (ls[2] + ls[3]);
        };
        // First against the current reference m, with no max: a weight past half's range (a score more than about
        // 16 above m, or m not yet set) rounds to infinity and makes the lane's sum infinite. Only then the tile's
        // max: m moves when it passes m by more than 8 (as in attn_kernel), O and l are rescaled and the weights
        // computed again (each at most 1 then). O / l does not depend on m.
        float lt = weights();
        if (__any(!(lt <= 3.0e38f))) {
            asm volatile("" ::: "memory");
            float mt[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float u = TAIL && !live(i) ? -INFINITY : x[i], w = TAIL && !live(i + 16) ? -INFINITY : x[i + 16];
                mt[i] = fmaxf(u, w);
            }
#pragma unroll
            for (int w = 8; w >= 1; w /= 2)
#pragma unroll
                for (int i = 0; i < w; ++i) mt[i] = fmaxf(mt[i], mt[i + w]);
            const float mx = (attn_pair_max(mt[0]) - (SAGE ? kScoreBias : 0.0f)) * f;
            if (mx > m + 8.0f) {
                const float mn = fmaxf(m, mx);
                alpha = __builtin_amdgcn_exp2f(m - mn);
                m = mn;
                l = l * alpha;
            }
            lt = weights();
        }
        l = l + lt;
    };
    using yes = std::true_type;
    using no = std::false_type;
    const bool ragged = S % kAttnRows != 0 && t0 + T == Tall;   // this range ends with the sequence's cut tile
    // Step t: refill the ring (tile t + NS - 1); the scores of tile t + 1 (DS); tile t's P v products (DPV) with the
    // softmax of tile t + 1 (independent of them) between them; O's rescale, if the softmax moved the reference; the
    // wait for tile t + 2 and one barrier. Tile j is read in steps j - 1 (K) and j (V^T); its stage is refilled at
    // step j + 1, after the barrier that ends step j.
    auto step = [&](int t, auto s_tag, auto pv_tag, auto tail_tag) {
        constexpr bool DS = decltype(s_tag)::value, DPV = decltype(pv_tag)::value;
        if (t >= 0) issue(t + NS - 1);
        if constexpr (DS) scores(t);
        if constexpr (DPV) pv(t);
        float alpha = 1.0f;
        if constexpr (DS) softmax(t, tail_tag, alpha);       // the compiler places it between the P v products
        if constexpr (DPV) {
            if (alpha != 1.0f) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) o[dt] = o[dt] * alpha;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) pb[u] = pn[u];
        wait_vm<LATER>();                                      // tile t + 2 is in (the barrier publishes it)
        lds_barrier();
    };

    // q's fragments and the scales are in before the first direct load: the compiler's own wait counts then see
    // nothing in flight inside the loop (the direct loads are not counted by it)
    wait_vm<0>();
    for (int t = 0; t < NS - 1; ++t) issue(t);
    wait_vm<(NS - 2) * (KI + VI)>();
    lds_barrier();                                             // tile 0 is in; qmax is written
    if constexpr (SAGE) {
        if (P.qraw) {
            // q's codes (attn_qk_prep_vec_kernel's arithmetic): the 64-row block's max over both wavefronts
            const float m = fmaxf(qm, qmax[wave ^ 1]);
            const float inv = m > 0.0f ? 127.0f / m : 0.0f;
#pragma unroll
            for (int kk = 0; kk < NQF; ++kk) {
                v4i_a w;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t b = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float cc = fminf(fmaxf(roundf(qx[kk * FR + 4 * i + e] * inv), -127.0f), 127.0f);
                        b |= (uint32_t) ((int) cc & 255) << (8 * e);
                    }
                    w[i] = (int) b;
                }
                qf[kk] = w;
            }
            fq = m / 127.0f * P.c;
        }
    }
    if (T == 1 && ragged) step(-1, yes{}, no{}, yes{});
    else step(-1, yes{}, no{}, no{});
    int t = 0;
    for (; t < T - 2; ++t) step(t, yes{}, yes{}, no{});
    if (t == T - 2) {                                          // the scores of the last tile
        if (ragged) step(t, yes{}, yes{}, yes{});
        else step(t, yes{}, yes{}, no{});
        ++t;
    }
    step(t, no{}, yes{}, no{});                                // step T - 1: the last P v products
    wait_vm<0>();                                              // no direct load may land after the block ends

    // ---- a split block: O, m and l of its key range for attn_merge_kernel ----
    if (slot >= 0) {
        const int64_t row = (int64_t) slot * kAttnPPQ + 32 * wave + ql;
        float* po = P.po + row * DK;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
                *reinterpret_cast<float4*>(po + 32 * dt + 8 * gq + 4 * hl) =
                    make_float4(o[dt][4 * gq], o[dt][4 * gq + 1], o[dt][4 * gq + 2], o[dt][4 * gq + 3]);
        const float lsum = attn_pair_sum(l);                   // m is the same in both lanes of the query
        if (hl == 0) *reinterpret_cast<float2*>(P.pml + 2 * row) = make_float2(m, lsum);
        return;
    }

    // ---- out = O / l, rounded to half, in out's type ----
    // Through LDS, so that the stores are whole rows: each wavefront stages its 32 queries, 256 bytes of features a
    // row per pass (all 128 features of a 16-bit out, 64 of a float32 one), into an area of its own in the ring
    // (free once every wavefront is past its last P v products), then reads it back as 16-byte chunks, four rows an
    // instruction.
    const float inv = 1.0f / attn_pair_sum(l);
    lds_barrier();
    constexpr int OPITCH = 256 + 16;                           // bytes a staged row (16 of pad: rows on other banks)
    static_assert(8 * 32 * OPITCH <= NS * STAGE, "the output staging fits in the ring");
    int8_t* ost = lds + wave * 32 * OPITCH;
    auto store = [&](auto dt_tag) {
        constexpr int OUT = decltype(dt_tag)::value;
        constexpr int esz = OUT == H3S_F32 ? 4 : 2;
        constexpr int FP = 256 / esz, NPASS = DK / FP, DTP = FP / 32;   // features, passes, o[] registers a pass
#pragma unroll
        for (int pass = 0; pass < NPASS; ++pass) {
#pragma unroll
            for (int d = 0; d < DTP; ++d)
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    // registers 4 gq .. 4 gq + 3 of o[dt]: features 32 dt + 8 gq + 4 hl + (0..3)
                    const int dt = pass * DTP + d;
                    float v[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = round_f16(o[dt][4 * gq + i] * inv);
                    int8_t* at = ost + ql * OPITCH + (32 * d + 8 * gq + 4 * hl) * esz;
                    if constexpr (OUT == H3S_F32) *reinterpret_cast<float4*>(at) = make_float4(v[0], v[1], v[2], v[3]);
                    else if constexpr (OUT == H3S_BF16) *reinterpret_cast<uint2*>(at) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
                    else *reinterpret_cast<uint2*>(at) = make_uint2(pack_f16(v[0], v[1]), pack_f16(v[2], v[3]));
                }
            wave_lds_sync();
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int ch = lane + 64 * k, r = ch / 16, c = ch % 16;
                const uint4 val = *reinterpret_cast<const uint4*>(ost + r * OPITCH + 16 * c);
                const int64_t qr = q0 + r;
                if (qr < S) *reinterpret_cast<uint4*>(reinterpret_cast<char*>(P.out) + ((qr * P.H + h) * DK + pass * FP) * esz + 16 * c) = val;
            }
            wave_lds_sync();
        }
    };
    if (P.out_dt == H3S_F32) store(std::integral_constant<int, H3S_F32>{});
    else if (P.out_dt == H3S_BF16) store(std::integral_constant<int, H3S_BF16>{});
    else store(std::integral_constant<int, H3S_F16>{});
}

// The split blocks' results combined: per query, M = max m_s, O = sum 2^(m_s - M) O_s, l = sum 2^(m_s - M) l_s,
// out = O / l rounded to half, in out's type (as the pipelined kernel's own epilogue). One thread a query and four
// features of the DK = 128.
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs P, int64_t tail) {
    constexpr int DK = 128;
    const int64_t id = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const int f0 = 4 * (int) (id % (DK / 4));
    const int64_t qq = id / (DK / 4);                          // query row among the split blocks' query blocks
    if (qq >= tail * kAttnPPQ) return;
    const int64_t tb = qq / kAttnPPQ, ob = P.nfull + tb, h = ob / P.nqb, qi = (ob % P.nqb) * kAttnPPQ + qq % kAttnPPQ;
    if (qi >= P.S) return;
    float M = -INFINITY;
    for (int s = 0; s < P.nsplit; ++s) M = fmaxf(M, P.pml[2 * ((tb * P.nsplit + s) * kAttnPPQ + qq % kAttnPPQ)]);
    float l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < P.nsplit; ++s) {
        const int64_t row = (tb * P.nsplit + s) * kAttnPPQ + qq % kAttnPPQ;
        const float2 ml = *reinterpret_cast<const float2*>(P.pml + 2 * row);
        const float w = __builtin_amdgcn_exp2f(ml.x - M);
        const float4 x = *reinterpret_cast<const float4*>(P.po + row * DK + f0);
        l = __builtin_fmaf(w, ml.y, l);
        o[0] = __builtin_fmaf(w, x.x, o[0]); o[1] = __builtin_fmaf(w, x.y, o[1]);
        o[2] = __builtin_fmaf(w, x.z, o[2]); o[3] = __builtin_fmaf(w, x.w, o[3]);
    }
    const float inv = 1.0f / l;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = round_f16(o[i] * inv);
    const int esz = P.out_dt == H3S_F32 ? 4 : 2;
    char* at = reinterpret_cast<char*>(P.out) + ((qi * P.H + h) * DK + f0) * esz;
    if (P.out_dt == H3S_F32) *reinterpret_cast<float4*>(at) = make_float4(v[0], v[1], v[2], v[3]);
    else if (P.out_dt == H3S_BF16) *reinterpret_cast<uint2*>(at) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    else *reinterpret_cast<uint2*>(at) = make_uint2(pack_f16(v[0], v[1]), pack_f16(v[2], v[3]));
}

}  // namespace h3
