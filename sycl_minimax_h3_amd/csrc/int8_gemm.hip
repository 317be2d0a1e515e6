// int8_gemm.hip - the int8 GEMM of h3s_int8_linear (kernels/h3sycl.cpp:576-631) on gfx950's i8 matrix cores, with
// the per-token x per-channel dequant (+ bias, + activation) in the epilogue, and h3s_int8_linear itself
// (quantizer, then this GEMM).
//
//   acc[m, n] = sum_k q[m, k] w[n, k]                  exact int32 (|acc| <= K 128 128 = 2^26 at K = 4096)
//   one weight scale:  out = acc * fl(s[m] * wscale[0])  (the row factor the reference folds first, h3sycl.cpp:576)
//   N weight scales:   out = (acc * s[m]) * wscale[n]    (the post-op order of h3sycl.cpp:588-602)
//   then + bias[n], then the activation, rounded once to out_dt.
//
// Tiles: a 256-thread workgroup computes a 256 x 256 block of out; its four waves (2 x 2) 128 x 128 each, as 4 x 4
// v_mfma_i32_32x32x32_i8 tiles. K advances 64 bytes a step through LDS (A and W both K-contiguous, rows padded to 80
// bytes so the 16-byte fragment reads of 32 consecutive rows hit distinct banks); the next step's tile is loaded
// into registers while the matrix cores work on this one.
#include "common.h"

namespace h3 {

constexpr int kBM = 256, kBN = 256, kBK = 64, kPitch = 80;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <int ACT, int PER_N>
__global__ __launch_bounds__(256) void gemm_i8_kernel(const int8_t* __restrict__ A, const float* __restrict__ sA, int64_t M,
                                                      int64_t K, const int8_t* __restrict__ W, int64_t N,
                                                      const float* __restrict__ ws, const float* __restrict__ bias,
                                                      void* __restrict__ out, int out_dt, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int8_t As[kBM * kPitch];
    __shared__ __attribute__((aligned(16))) int8_t Bs[kBN * kPitch];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t) (blockIdx.x / tiles_n) * kBM, n0 = (int64_t) (blockIdx.x % tiles_n) * kBN;

    // global -> register staging: thread t moves 16-byte pieces t + 256 i (i < 4) of each 256 x 64 tile; rows past
    // M or N read the last row again (their products land in rows / columns that are not stored)
    const int8_t* pa[4];
    const int8_t* pb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int id = tid + 256 * i, r = id >> 2, c16 = id & 3;
        const int64_t ma = m0 + r < M ? m0 + r : M - 1, nb = n0 + r < N ? n0 + r : N - 1;
        pa[i] = A + ma * K + c16 * 16;
        pb[i] = W + nb * K + c16 * 16;
    }
    uint4 ga[4], gb[4];
    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ga[i] = *reinterpret_cast<const uint4*>(pa[i] + k0);
            gb[i] = *reinterpret_cast<const uint4*>(pb[i] + k0);
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = tid + 256 * i, r = id >> 2, c16 = id & 3;
            *reinterpret_cast<uint4*>(As + r * kPitch + c16 * 16) = ga[i];
            *reinterpret_cast<uint4*>(Bs + r * kPitch + c16 * 16) = gb[i];
        }
    };

    v16i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v16i) 0;

    const int64_t nk = K / kBK;
    gload(0);
    sstore();
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32) {
            // lane l: row / column l % 32 of its 32 x 32 tile, 16 consecutive k from kk + 16 (l / 32)
            const int koff = kk + 16 * (lane >> 5);
            v4i a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const v4i*>(As + (wm * 128 + i * 32 + (lane & 31)) * kPitch + koff);
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const v4i*>(Bs + (wn * 128 + j * 32 + (lane & 31)) * kPitch + koff);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
        if (kt + 1 < nk) {
            sstore();
            __syncthreads();
        }
    }

    // epilogue: register r of a 32 x 32 tile holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + wn * 128 + j * 32 + (lane & 31);
        if (n >= N) continue;
        const float wsn = PER_N ? ws[n] : 0.0f;
        const float bn = bias ? bias[n] : 0.0f;
        const float ws0 = ws[0];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t m = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= M) continue;
                const float sr = sA[m];
                float v = PER_N ? (float) acc[i][j][r] * sr * wsn : (float) acc[i][j][r] * (sr * ws0);
                if (bias) v = v + bn;
                v = act<ACT>(v);
                const int64_t o = m * N + n;
                if (out_dt == H3S_F32) ((float*) out)[o] = v;
                else if (out_dt == H3S_BF16) ((uint16_t*) out)[o] = (uint16_t) pack_bf16(v, 0.0f);
                else ((uint16_t*) out)[o] = (uint16_t) pack_f16(v, 0.0f);
            }
    }
}

int launch_gemm(Ctx* c, const char* fn, const int8_t* q, const float* s, int64_t M, int64_t K, const int8_t* w, int64_t N,
                const float* wscale, int64_t n_wscale, const float* bias, int act_, void* out, int out_dt) {
    const int64_t tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
    if (tm * tn > 0x7fffffff) return fail(std::string(fn) + ": too many tiles");
    const unsigned grid = (unsigned) (tm * tn);
    const bool per_n = n_wscale > 1;
#define LG(ACT, PN) gemm_i8_kernel<ACT, PN><<<grid, 256, 0, c->stream>>>(q, s, M, K, w, N, wscale, bias, out, out_dt, (int) tn)
#define LA(ACT)                    \
    if (per_n) LG(ACT, 1);         \
    else LG(ACT, 0);
    if (act_ == H3S_ACT_SILU) { LA(H3S_ACT_SILU); }
    else if (act_ == H3S_ACT_GELU_TANH) { LA(H3S_ACT_GELU_TANH); }
    else { LA(H3S_ACT_NONE); }
#undef LA
#undef LG
    return launched(fn);
}

static int gemm_checks(const char* fn, int64_t K, int64_t N, int64_t n_wscale, int out_dt, const void* q, const void* w,
                       const void* out) {
    if (K % kBK != 0) return fail(std::string(fn) + ": K must be a multiple of 64");
    if (n_wscale != 1 && n_wscale != N) return fail(std::string(fn) + ": 1 or N weight scales");
    if (!dt_ok(out_dt)) return fail(std::string(fn) + ": unknown element type");
    if (!aligned16(q) || !aligned16(w)) return fail(std::string(fn) + ": q and w must be 16-byte aligned");
    if (!out) return fail(std::string(fn) + ": out is required");
    return 0;
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_int8_gemm_dequant(void* ctx, const int8_t* q, const float* s, int64_t M, int64_t K, const int8_t* w, int64_t N,
                                     const float* wscale, int64_t n_wscale, const float* bias, int act, void* out,
                                     int out_dt) try {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (gemm_checks("h3s_int8_gemm_dequant", K, N, n_wscale, out_dt, q, w, out)) return -1;
    if (act != H3S_ACT_NONE && act != H3S_ACT_SILU && act != H3S_ACT_GELU_TANH) return fail("h3s_int8_gemm_dequant: unknown activation");
    Ctx* c = ctx_of(ctx, "h3s_int8_gemm_dequant");
    if (!c) return -1;
    return launch_gemm(c, "h3s_int8_gemm_dequant", q, s, M, K, w, N, wscale, n_wscale, bias, act, out, out_dt);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_int8_linear(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N,
                               const float* wscale, int64_t n_wscale, const float* bias, void* out, int out_dt, int group) try {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    // kernels/h3sycl.h:83: the group is 0 or a power of 4, at most 256, dividing K
    if (group < 0 || (group > 0 && (group > 256 || K % group != 0 || (group & (group - 1)) != 0 || (__builtin_ctz((unsigned) group) & 1))))
        return fail("h3s_int8_linear: unsupported ConvRot group size (0, or a power of 4 at most 256 dividing K)");
    if (!dt_ok(x_dt)) return fail("h3s_int8_linear: unknown element type");
    if (gemm_checks("h3s_int8_linear", K, N, n_wscale, out_dt, x, w, out)) return -1;
    Ctx* c = ctx_of(ctx, "h3s_int8_linear");
    if (!c) return -1;
    // the quantized rows and their scales, a chunk of rows at a time (kernels/h3sycl.cpp:640-651)
    constexpr int64_t kRows = 65536;
    const int64_t rows = M < kRows ? M : kRows;
    int8_t* xq = c->grow(c->xq, c->xq_cap, (size_t) (rows * K));
    float* rs = c->grow(c->rs, c->rs_cap, (size_t) rows);
    if (!xq || !rs) return -1;
    const size_t xe = (size_t) elem_size(x_dt), oe = (size_t) elem_size(out_dt);
    for (int64_t r0 = 0; r0 < M; r0 += kRows) {
        const int64_t n = M - r0 < kRows ? M - r0 : kRows;
        if (launch_quantize(c, (const char*) x + (size_t) (r0 * K) * xe, x_dt, n, K, group, xq, rs)) return -1;
        if (launch_gemm(c, "h3s_int8_linear", xq, rs, n, K, w, N, wscale, n_wscale, bias, H3S_ACT_NONE,
                        (char*) out + (size_t) (r0 * N) * oe, out_dt))
            return -1;
    }
    return 0;
} catch (const std::exception& e) { return fail(e.what()); }
