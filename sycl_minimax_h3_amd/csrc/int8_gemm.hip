// int8_gemm.hip - the entry points of the int8 GEMM (kernel: gemm_impl.h): h3s_int8_gemm_dequant (quantized rows in,
// dequant + bias + activation epilogue), h3s_int8_linear (kernels/h3sycl.cpp:633-652: the quantizer, then the GEMM, a
// chunk of rows at a time, the quantized rows in the context's scratch) and h3s_int8_linear_noalloc (the same, the
// quantized rows in a fixed device array, for callers that cannot allocate).
#include <map>

#include "gemm_impl.h"

namespace h3 {

// ---- the fixed scratch of h3s_int8_linear_noalloc ----
// int8 codes of one row chunk (64 MiB), then the chunk's float32 row scales. Each device the library runs on holds
// its own copy until the process ends. Host code never hands the array's name to a kernel: in host code it stands for
// no device address. Its address on each device is looked up once (noalloc_setup, at context creation).
constexpr size_t kScratchCodes = (size_t) 64 << 20;
constexpr int64_t kScratchRows = 65536;
constexpr int64_t kScratchMaxK = 65536;             // features a row: every chunk then holds at least 1024 rows
static __device__ __align__(256) int8_t scratch[kScratchCodes + kScratchRows * sizeof(float)];

static std::mutex g_scratch_mu;
static std::map<int, void*> g_scratch_at;           // device -> the array's address there
static std::map<int, std::string> g_scratch_err;    // device -> why the lookup failed

int noalloc_setup(int device) {
    std::lock_guard<std::mutex> l(g_scratch_mu);
    if (g_scratch_at.count(device) || g_scratch_err.count(device)) return g_scratch_at.count(device) ? 0 : -1;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void) hipGetLastError();
        g_scratch_err[device] = std::string("the address of the fixed scratch on GPU ") + std::to_string(device) +
                                " could not be found: " + hipGetErrorString(e);
        return -1;
    }
    g_scratch_at[device] = p;
    return 0;
}

static void* scratch_on(int device, std::string& why) {
    std::lock_guard<std::mutex> l(g_scratch_mu);
    const auto it = g_scratch_at.find(device);
    if (it != g_scratch_at.end()) return it->second;
    const auto er = g_scratch_err.find(device);
    why = er != g_scratch_err.end() ? er->second : "the fixed scratch was not set up on GPU " + std::to_string(device);
    return nullptr;
}

// the GEMM of quantized rows, and (split last tiles) the merge of their parts; split_ok false: every tile whole (no
// scratch, for the allocation-free entry point)
int launch_gemm(Ctx* c, const char* fn, const int8_t* q, const float* s, int64_t M, int64_t K, const int8_t* w, int64_t N,
                const float* wscale, int64_t n_wscale, const float* bias, int act_, void* out, int out_dt, bool split_ok) {
    const int64_t tm = (M + kGemmBM - 1) / kGemmBM, tn = (N + kGemmBN - 1) / kGemmBN;
    if (tm * tn > 0x7fffffff || tm > 0x7fffffff || tn > 0x7fffffff) return fail(std::string(fn) + ": too many tiles");
    int main_tiles = (int) (tm * tn), split = 1;
    if (split_ok) gemm_plan_split(tm * tn, (K + kGemmBK - 1) / kGemmBK, c->cus, &main_tiles, &split);
    const int64_t tail = tm * tn - main_tiles;
    void* part = nullptr;
    if (split > 1) {
        part = c->scratch<int32_t>(Ctx::GEMM_PART, (size_t) (tail * split) * kGemmTileAcc);
        if (!part) return -1;
    }
    const GemmArgs P{q, s, M, K, w, N, wscale, bias, out, out_dt, (int) tm, (int) tn, K >= 12288 ? 4 : 8, main_tiles, split, part};
    const unsigned grid = (unsigned) (main_tiles + tail * split);
    const bool per_n = n_wscale > 1;
    const unsigned mgrid = (unsigned) (tail * kGemmMergeBlocks);
    // the merge for one activation, weight-scale kind, output type and bias
#define LM(ACT, PN)                                                                                                  \
    if (split > 1) {                                                                                                 \
        if (out_dt == H3S_BF16) {                                                                                    \
            if (bias) gemm_merge_kernel<GEMM_I8, ACT, PN, false, H3S_BF16, true><<<mgrid, 256, 0, c->stream>>>(P);    \
            else gemm_merge_kernel<GEMM_I8, ACT, PN, false, H3S_BF16, false><<<mgrid, 256, 0, c->stream>>>(P);       \
        } else if (out_dt == H3S_F16) {                                                                              \
            if (bias) gemm_merge_kernel<GEMM_I8, ACT, PN, false, H3S_F16, true><<<mgrid, 256, 0, c->stream>>>(P);     \
            else gemm_merge_kernel<GEMM_I8, ACT, PN, false, H3S_F16, false><<<mgrid, 256, 0, c->stream>>>(P);        \
        } else {                                                                                                     \
            if (bias) gemm_merge_kernel<GEMM_I8, ACT, PN, false, H3S_F32, true><<<mgrid, 256, 0, c->stream>>>(P);     \
            else gemm_merge_kernel<GEMM_I8, ACT, PN, false, H3S_F32, false><<<mgrid, 256, 0, c->stream>>>(P);        \
        }                                                                                                            \
    }
#define LG(ACT, PN)                                                        \
    {                                                                      \
        gemm_i8_kernel<ACT, PN><<<grid, kGemmThreads, 0, c->stream>>>(P);  \
        LM(ACT, PN)                                                        \
    }
#define LA(ACT)                    \
    if (per_n) LG(ACT, true)       \
    else LG(ACT, false)
    if (act_ == H3S_ACT_SILU) { LA(H3S_ACT_SILU); }
    else if (act_ == H3S_ACT_GELU_TANH) { LA(H3S_ACT_GELU_TANH); }
    else { LA(H3S_ACT_NONE); }
#undef LA
#undef LG
#undef LM
    return launched(fn);
}

static int gemm_checks(const char* fn, int64_t K, int64_t N, int64_t n_wscale, int out_dt, const void* q, const void* w,
                       const void* out) {
    if (K % 64 != 0) return fail(std::string(fn) + ": K must be a multiple of 64");
    if (K >= (int64_t) 1 << 24) return fail(std::string(fn) + ": K must be below 2^24");
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
    return launch_gemm(c, "h3s_int8_gemm_dequant", q, s, M, K, w, N, wscale, n_wscale, bias, act, out, out_dt, true);
} catch (const std::exception& e) { return fail(e.what()); }

namespace h3 {

// the checks both int8 linear entry points share; 0 or -1 with the reason
static int linear_checks(const char* fn, const void* x, int x_dt, int64_t K, int64_t N, const int8_t* w, int64_t n_wscale,
                         void* out, int out_dt, int group) {
    // kernels/h3sycl.h:83: the group is 0 or a power of 4, at most 256, dividing K
    if (group < 0 || (group > 0 && (group > 256 || K % group != 0 || (group & (group - 1)) != 0 || (__builtin_ctz((unsigned) group) & 1))))
        return fail(std::string(fn) + ": unsupported ConvRot group size (0, or a power of 4 at most 256 dividing K)");
    if (!dt_ok(x_dt)) return fail(std::string(fn) + ": unknown element type");
    return gemm_checks(fn, K, N, n_wscale, out_dt, x, w, out);
}

// the quantizer, then the GEMM, rows at a time into xq [rows, K] and rs [rows]
static int linear_chunks(Ctx* c, const char* fn, const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N,
                         const float* wscale, int64_t n_wscale, const float* bias, void* out, int out_dt, int group, int8_t* xq,
                         float* rs, int64_t rows, bool timed, bool split_ok) {
    const size_t xe = (size_t) elem_size(x_dt), oe = (size_t) elem_size(out_dt);
    for (int64_t r0 = 0; r0 < M; r0 += rows) {
        const int64_t n = M - r0 < rows ? M - r0 : rows;
        PhaseTimer t(c, timed);
        t.mark();
        if (launch_quantize(c, (const char*) x + (size_t) (r0 * K) * xe, x_dt, n, K, group, xq, rs)) return -1;
        t.mark();
        if (launch_gemm(c, fn, xq, rs, n, K, w, N, wscale, n_wscale, bias, H3S_ACT_NONE, (char*) out + (size_t) (r0 * N) * oe,
                        out_dt, split_ok))
            return -1;
        t.mark();
        const std::vector<float> ms = t.elapsed();
        if (ms.size() == 2) {
            c->lin_ms[0] += ms[0];
            c->lin_ms[1] += ms[1];
            ++c->lin_chunks;
        }
    }
    return 0;
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_int8_linear(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N,
                               const float* wscale, int64_t n_wscale, const float* bias, void* out, int out_dt, int group) try {
    const char* fn = "h3s_int8_linear";
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (linear_checks(fn, x, x_dt, K, N, w, n_wscale, out, out_dt, group)) return -1;
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    // the quantized rows and their scales in the context's scratch, a chunk of rows at a time
    // (kernels/h3sycl.cpp:640-651)
    constexpr int64_t kRows = 65536;
    const int64_t rows = M < kRows ? M : kRows;
    int8_t* xq = c->scratch<int8_t>(Ctx::LIN_CODES, (size_t) (rows * K));
    float* rs = c->scratch<float>(Ctx::LIN_SCALES, (size_t) rows);
    if (!xq || !rs) return -1;
    return linear_chunks(c, fn, x, x_dt, M, K, w, N, wscale, n_wscale, bias, out, out_dt, group, xq, rs, rows, true, true);
} catch (const std::exception& e) { return fail(e.what()); }

// h3s_int8_linear with the quantized rows in the fixed device array: no allocation, any M (in chunks of at most
// 65536 rows and 64 MiB of codes), K at most 65536. Calls on one GPU share its array: calls that overlap on one GPU
// (two streams, two contexts) race.
H3S_EXPORT int h3s_int8_linear_noalloc(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N,
                                       const float* wscale, int64_t n_wscale, const float* bias, void* out, int out_dt,
                                       int group) try {
    const char* fn = "h3s_int8_linear_noalloc";
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (K > kScratchMaxK)
        return fail(std::string(fn) + ": rows of " + std::to_string(K) + " features pass the fixed scratch's limit of " +
                    std::to_string(kScratchMaxK));
    if (linear_checks(fn, x, x_dt, K, N, w, n_wscale, out, out_dt, group)) return -1;
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    std::string why;
    char* base = static_cast<char*>(scratch_on(c->device, why));
    if (!base) return fail(std::string(fn) + ": " + why);
    const int64_t by_codes = (int64_t) (kScratchCodes / (size_t) K);
    const int64_t rows = by_codes < kScratchRows ? by_codes : kScratchRows;
    return linear_chunks(c, fn, x, x_dt, M, K, w, N, wscale, n_wscale, bias, out, out_dt, group, reinterpret_cast<int8_t*>(base),
                         reinterpret_cast<float*>(base + kScratchCodes), rows, false, false);
} catch (const std::exception& e) { return fail(e.what()); }
