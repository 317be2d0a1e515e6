// linear.hip - the plain (float) linear layers of kernels/h3sycl.h:87-93: h3s_linear (out = x w^T + bias),
// h3s_linear_acc (out += x w^T + bias, a LoRA's second factor) and h3s_scale_rows (kernels/h3sycl.cpp:656-739).
// bfloat16 and half operands with K a multiple of 32 run on the matrix cores in gemm_impl.h's pipeline
// (gemm_f16_kernel): float32 accumulation, and the epilogue adds the bias (and the old output) in float32 and rounds
// once to the output type, as the reference's matmul post-ops do, with no intermediate in memory. Every other call
// (float32 operands, other K, unaligned rows) runs on rocBLAS (a plain library GEMM, float32 accumulation, on the
// context's stream) into a float32 scratch, a chunk of rows at a time, and the same epilogue as a kernel of its own.
#include <rocblas/rocblas.h>

#include "gemm_impl.h"

namespace h3 {

void release_blas(Ctx* c) {
    if (c->blas) (void) rocblas_destroy_handle((rocblas_handle) c->blas);
    c->blas = nullptr;
}

static rocblas_handle blas_of(Ctx* c) {
    if (!c->blas) {
        rocblas_handle h = nullptr;
        count_alloc();
        if (rocblas_create_handle(&h) != rocblas_status_success) { set_error("rocBLAS: no handle"); return nullptr; }
        if (rocblas_set_stream(h, c->stream) != rocblas_status_success) {
            (void) rocblas_destroy_handle(h);
            set_error("rocBLAS: could not bind the context's stream");
            return nullptr;
        }
        c->blas = h;
    }
    return (rocblas_handle) c->blas;
}

static rocblas_datatype blas_type(int dt) {
    return dt == H3S_F32 ? rocblas_datatype_f32_r : dt == H3S_F16 ? rocblas_datatype_f16_r : rocblas_datatype_bf16_r;
}

template <int DT> __device__ __forceinline__ float lin_load(const void* p, int64_t i) {
    if constexpr (DT == H3S_F32) return ((const float*) p)[i];
    else if constexpr (DT == H3S_BF16) return bf16_lo(((const uint16_t*) p)[i]);
    else return f16_lo(((const uint16_t*) p)[i]);
}
template <int DT> __device__ __forceinline__ void lin_store(void* p, int64_t i, float v) {
    if constexpr (DT == H3S_F32) ((float*) p)[i] = v;
    else if constexpr (DT == H3S_BF16) ((uint16_t*) p)[i] = (uint16_t) pack_bf16(v, 0.0f);
    else ((uint16_t*) p)[i] = (uint16_t) pack_f16(v, 0.0f);
}

// out[r, n] = round(acc[r, n] [+ bias[n]] [+ out[r, n]]) over rows [0, M)
template <int DT, bool ACC>
__global__ __launch_bounds__(256) void lin_epilogue_kernel(const float* __restrict__ acc, int64_t M, int64_t N,
                                                           const float* __restrict__ bias, void* out) {
    const int64_t n = M * N;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t) gridDim.x * 256) {
        float v = acc[i];
        if (bias) v = v + bias[i % N];
        if constexpr (ACC) v = v + lin_load<DT>(out, i);
        lin_store<DT>(out, i, v);
    }
}

template <int DT>
__global__ __launch_bounds__(256) void scale_rows_kernel(void* x, int64_t M, int64_t C, const float* __restrict__ s) {
    const int64_t n = M * C;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t) gridDim.x * 256)
        lin_store<DT>(x, i, lin_load<DT>(x, i) * s[i / C]);
}

static unsigned grid_of(int64_t n, const Ctx& c) {
    const int64_t b = (n + 255) / 256, cap = (int64_t) c.cus * 16;
    return (unsigned) (b < cap ? (b > 0 ? b : 1) : cap);
}

template <bool ACC>
static int launch_epilogue(Ctx* c, const float* acc, int64_t M, int64_t N, const float* bias, void* out, int out_dt) {
    const unsigned g = grid_of(M * N, *c);
    switch (out_dt) {
        case H3S_F32: lin_epilogue_kernel<H3S_F32, ACC><<<g, 256, 0, c->stream>>>(acc, M, N, bias, out); break;
        case H3S_F16: lin_epilogue_kernel<H3S_F16, ACC><<<g, 256, 0, c->stream>>>(acc, M, N, bias, out); break;
        default: lin_epilogue_kernel<H3S_BF16, ACC><<<g, 256, 0, c->stream>>>(acc, M, N, bias, out); break;
    }
    return 0;
}

// whether gemm_f16_kernel takes the product: 16-bit operands whose rows are whole 64-byte units (the pipeline's
// half K step) and start on 16-byte boundaries (out too), K * 2 below 2^24 bytes, tile counts within 32 bits
static bool mfma_takes(int dt, const void* x, const void* w, const void* out, int64_t M, int64_t K, int64_t N) {
    const int64_t tm = (M + kGemmBM - 1) / kGemmBM, tn = (N + kGemmBN - 1) / kGemmBN;
    return (dt == H3S_BF16 || dt == H3S_F16) && K % 32 == 0 && 2 * K < ((int64_t) 1 << 24) && aligned16(x) &&
           aligned16(w) && aligned16(out) && tm * tn <= 0x7fffffff;
}
// the merge of the split last tiles for operand type OP (out_dt: the output type; ACC: h3s_linear_acc, out in dt)
template <int OP, bool ACC>
static void merge_f16(Ctx* c, const GemmArgs& P, unsigned mgrid) {
    const bool b = P.bias != nullptr;
    if (P.out_dt == H3S_BF16) {
        if (b) gemm_merge_kernel<OP, H3S_ACT_NONE, false, ACC, H3S_BF16, true><<<mgrid, 256, 0, c->stream>>>(P);
        else gemm_merge_kernel<OP, H3S_ACT_NONE, false, ACC, H3S_BF16, false><<<mgrid, 256, 0, c->stream>>>(P);
    } else if (P.out_dt == H3S_F16) {
        if (b) gemm_merge_kernel<OP, H3S_ACT_NONE, false, ACC, H3S_F16, true><<<mgrid, 256, 0, c->stream>>>(P);
        else gemm_merge_kernel<OP, H3S_ACT_NONE, false, ACC, H3S_F16, false><<<mgrid, 256, 0, c->stream>>>(P);
    } else if constexpr (!ACC) {
        if (b) gemm_merge_kernel<OP, H3S_ACT_NONE, false, false, H3S_F32, true><<<mgrid, 256, 0, c->stream>>>(P);
        else gemm_merge_kernel<OP, H3S_ACT_NONE, false, false, H3S_F32, false><<<mgrid, 256, 0, c->stream>>>(P);
    }
}
static int linear_mfma(Ctx* c, const char* fn, const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N,
                       const float* bias, void* out, int out_dt, bool acc) {
    const int64_t tm = (M + kGemmBM - 1) / kGemmBM, tn = (N + kGemmBN - 1) / kGemmBN, kb = 2 * K;
    int main_tiles = (int) (tm * tn), split = 1;
    gemm_plan_split(tm * tn, (kb + kGemmBK - 1) / kGemmBK, c->cus, &main_tiles, &split);
    const int64_t tail = tm * tn - main_tiles;
    void* part = nullptr;
    if (split > 1) {
        part = c->scratch<float>(Ctx::GEMM_PART, (size_t) (tail * split) * kGemmTileAcc);
        if (!part) return -1;
    }
    const GemmArgs P{(const int8_t*) x, nullptr, M, kb, (const int8_t*) w, N, nullptr, bias, out, out_dt, (int) tm, (int) tn,
                     kb >= 12288 ? 4 : 8, main_tiles, split, part};
    const unsigned grid = (unsigned) (main_tiles + tail * split), mgrid = (unsigned) (tail * kGemmMergeBlocks);
    if (dt == H3S_BF16) {
        if (acc) gemm_f16_kernel<GEMM_BF16, true><<<grid, kGemmThreads, 0, c->stream>>>(P);
        else gemm_f16_kernel<GEMM_BF16, false><<<grid, kGemmThreads, 0, c->stream>>>(P);
        if (split > 1) { if (acc) merge_f16<GEMM_BF16, true>(c, P, mgrid); else merge_f16<GEMM_BF16, false>(c, P, mgrid); }
    } else {
        if (acc) gemm_f16_kernel<GEMM_F16, true><<<grid, kGemmThreads, 0, c->stream>>>(P);
        else gemm_f16_kernel<GEMM_F16, false><<<grid, kGemmThreads, 0, c->stream>>>(P);
        if (split > 1) { if (acc) merge_f16<GEMM_F16, true>(c, P, mgrid); else merge_f16<GEMM_F16, false>(c, P, mgrid); }
    }
    return launched(fn);
}

// the product x [M, K] . w^T (w [N, K]), both in dt, into out (or out +=): on the matrix cores, or on rocBLAS a
// chunk of rows at a time
static int linear(Ctx* c, const char* fn, const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N,
                  const float* bias, void* out, int out_dt, bool acc) {
    if (K > 0x7fffffff || N > 0x7fffffff) return fail(std::string(fn) + ": K and N must be below 2^31");
    if (mfma_takes(dt, x, w, out, M, K, N)) return linear_mfma(c, fn, x, dt, M, K, w, N, bias, out, out_dt, acc);
    rocblas_handle h = blas_of(c);
    if (!h) return -1;
    // rows a chunk: the float32 product of a chunk takes at most 256 MiB (and at most 8192 rows, as the reference)
    int64_t rows = (int64_t) (256 << 20) / (N * 4);
    rows = rows < 1 ? 1 : rows > 8192 ? 8192 : rows;
    rows = rows < M ? rows : M;
    float* tmp = c->scratch<float>(Ctx::LIN_F32, (size_t) (rows * N));
    if (!tmp) return -1;
    const size_t xe = (size_t) elem_size(dt), oe = (size_t) elem_size(out_dt);
    const float one = 1.0f, zero = 0.0f;
    for (int64_t r0 = 0; r0 < M; r0 += rows) {
        const int64_t m = M - r0 < rows ? M - r0 : rows;
        // column-major view: tmp^T [N, m] = w [N, K] (stored as K x N, transposed) . x^T [K, m]
        const rocblas_status st = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int) N,
                                                  (rocblas_int) m, (rocblas_int) K, &one, w, blas_type(dt), (rocblas_int) K,
                                                  (const char*) x + (size_t) (r0 * K) * xe, blas_type(dt), (rocblas_int) K,
                                                  &zero, tmp, rocblas_datatype_f32_r, (rocblas_int) N, tmp,
                                                  rocblas_datatype_f32_r, (rocblas_int) N, rocblas_datatype_f32_r,
                                                  rocblas_gemm_algo_standard, 0, 0);
        if (st != rocblas_status_success)
            return fail(std::string(fn) + ": rocBLAS gemm_ex failed (" + rocblas_status_to_string(st) + ")");
        char* o = (char*) out + (size_t) (r0 * N) * oe;
        if (acc) launch_epilogue<true>(c, tmp, m, N, bias, o, out_dt);
        else launch_epilogue<false>(c, tmp, m, N, bias, o, out_dt);
        if (launched(fn)) return -1;
    }
    return 0;
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_linear(void* ctx, const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N, const float* bias,
                          void* out, int out_dt) try {
    const char* fn = "h3s_linear";
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (!dt_ok(dt) || !dt_ok(out_dt)) return fail(std::string(fn) + ": unknown element type");
    if (!x || !w || !out) return fail(std::string(fn) + ": x, w and out are required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return linear(c, fn, x, dt, M, K, w, N, bias, out, out_dt, false);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_linear_acc(void* ctx, const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N,
                              const float* bias, void* out) try {
    const char* fn = "h3s_linear_acc";
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (!dt_ok(dt)) return fail(std::string(fn) + ": unknown element type");
    if (!x || !w || !out) return fail(std::string(fn) + ": x, w and out are required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return linear(c, fn, x, dt, M, K, w, N, bias, out, dt, true);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_scale_rows(void* ctx, void* x, int dt, int64_t M, int64_t C, const float* s) try {
    const char* fn = "h3s_scale_rows";
    if (M <= 0 || C <= 0) return 0;
    if (!dt_ok(dt)) return fail(std::string(fn) + ": unknown element type");
    if (!x || !s) return fail(std::string(fn) + ": x and s are required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    const unsigned g = grid_of(M * C, *c);
    switch (dt) {
        case H3S_F32: scale_rows_kernel<H3S_F32><<<g, 256, 0, c->stream>>>(x, M, C, s); break;
        case H3S_F16: scale_rows_kernel<H3S_F16><<<g, 256, 0, c->stream>>>(x, M, C, s); break;
        default: scale_rows_kernel<H3S_BF16><<<g, 256, 0, c->stream>>>(x, M, C, s); break;
    }
    return launched(fn);
} catch (const std::exception& e) { return fail(e.what()); }
