// quant.hip - the entry points of the row quantizer: h3s_norm_quant (rms_norm_mod -> the reference's bf16
// scratch h -> int8_linear's quantizer, in one pass), h3s_swiglu_quant (h3s_swiglu -> the MLP's scratch act ->
// fc2's quantizer, in one pass) and launch_quantize (h3s_int8_linear's quantizer). The kernel is quant_impl.h,
// instantiated per input type in quant_bf16.hip, quant_f16.hip and quant_f32.hip.
#include <cmath>

#include "quant_impl.h"

namespace h3 {

template <int XDT> int quant_launch(Ctx*, const char*, const QuantArgs&, int, RowPlan);
extern template int quant_launch<H3S_BF16>(Ctx*, const char*, const QuantArgs&, int, RowPlan);
extern template int quant_launch<H3S_F16>(Ctx*, const char*, const QuantArgs&, int, RowPlan);
extern template int quant_launch<H3S_F32>(Ctx*, const char*, const QuantArgs&, int, RowPlan);

static int dispatch(Ctx* c, const char* fn, int x_dt, const QuantArgs& A, int mode, RowPlan p) {
    switch (x_dt) {
        case H3S_BF16: return quant_launch<H3S_BF16>(c, fn, A, mode, p);
        case H3S_F16: return quant_launch<H3S_F16>(c, fn, A, mode, p);
        default: return quant_launch<H3S_F32>(c, fn, A, mode, p);
    }
}

// the rotation arguments of h3s_norm_quant and h3s_swiglu_quant; 0 or -1 (a failure with the reason)
static int rot_checks(const char* fn, int rot, int group, int64_t C, int V);

static bool is_pow2(int g) { return g > 0 && (g & (g - 1)) == 0; }
static float inv_sqrt_group(int g) { return (float) (1.0 / std::sqrt((double) g)); }
static const char* too_long = ": rows longer than 2048 16-byte vectors (16384 16-bit or 8192 float32 features) are not supported";

int launch_quantize(Ctx* c, const void* x, int x_dt, int64_t M, int64_t K, int group, int8_t* q, float* s) {
    const char* fn = "h3s_int8_linear";
    const int V = vec_of(x_dt);
    if (K % V != 0) return fail(std::string(fn) + ": K must be whole 16-byte vectors");
    const RowPlan p = row_plan(K / V);
    if (!p.L) return fail(std::string(fn) + too_long);
    const QuantArgs A{x, M, K, nullptr, 0.0f, nullptr, nullptr, nullptr, H3S_F32, H3S_F32,
                      group > 0 ? H3S_ROT_REGULAR : H3S_ROT_NONE, group, group > 0 ? inv_sqrt_group(group) : 1.0f, q, s};
    return dispatch(c, fn, x_dt, A, QUANT_RAW, p);
}

// h3s_rms_norm_mod on the one-wavefront-a-row layout, for the shapes it takes (bfloat16 rows and out of the model's
// hidden width, a weight, float32 tables or none): 0 or -1 when it ran, 1 when the shape is not one it takes.
int launch_norm_out(Ctx* c, const char* fn, const void* x, int x_dt, int64_t M, int64_t C, const float* w, float eps,
                    const int32_t* rows, const float* scale, const float* shift, void* out, int out_dt) {
    if (x_dt != H3S_BF16 || out_dt != H3S_BF16 || !w || M < c->quant_wave_min) return 1;
    QuantArgs A{x, M, C, w, eps, rows, scale, shift, H3S_F32, H3S_BF16, H3S_ROT_NONE, 0, 1.0f, nullptr, nullptr};
    A.h = out;
    const int f = ROW_W | (scale ? ROW_TAB | ROW_TAB32 : 0) | ROW_OUTH;
    if (!quant_wave_model_takes(A, f)) return 1;
    return quant_launch<H3S_BF16>(c, fn, A, QUANT_NORM_OUT, row_plan(C / 8));
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_norm_quant(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps,
                              const int32_t* rows, const void* scale, const void* shift, int tab_dt, int h_dt, int rot,
                              int group, int8_t* q, float* s) try {
    if (M <= 0 || C <= 0) return 0;
    const char* fn = "h3s_norm_quant";
    if (!dt_ok(x_dt) || !dt_ok(h_dt) || !dt_ok(tab_dt)) return fail(std::string(fn) + ": unknown element type");
    const int V = vec_of(x_dt);
    if (C % V != 0) return fail(std::string(fn) + ": C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors per row)");
    for (const void* p : {x, (const void*) weight, scale, shift, (const void*) q})
        if (p && !aligned16(p)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    if (!x || !q || !s) return fail(std::string(fn) + ": x, q and s are required");
    if (rot_checks(fn, rot, group, C, V)) return -1;
    const bool mod = scale && shift;
    if (mod && tab_dt != H3S_F32 && tab_dt != H3S_BF16) return fail(std::string(fn) + ": tables are float32 or bfloat16");
    const RowPlan p = row_plan(C / V);
    if (!p.L) return fail(std::string(fn) + too_long);
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    const QuantArgs A{x, M, C, weight, eps, rows, mod ? scale : nullptr, mod ? shift : nullptr, tab_dt, h_dt, rot,
                      rot != H3S_ROT_NONE ? group : 0, rot != H3S_ROT_NONE ? inv_sqrt_group(group) : 1.0f, q, s};
    return dispatch(c, fn, x_dt, A, QUANT_NORM, p);
} catch (const std::exception& e) { return fail(e.what()); }

// h3s_int8_linear's first pass on its own (kernels/h3sycl.cpp:404-474, 521-575): x [M, K] rotated per group (0: none,
// else the regular Hadamard of that size) and quantized to codes q [M, K] and row scales s [M].
H3S_EXPORT int h3s_int8_quantize(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, int group, int8_t* q, float* s) try {
    if (M <= 0 || K <= 0) return 0;
    const char* fn = "h3s_int8_quantize";
    if (!dt_ok(x_dt)) return fail(std::string(fn) + ": unknown element type");
    if (group < 0 || (group > 0 && (group > 256 || K % group != 0 || (group & (group - 1)) != 0 || (__builtin_ctz((unsigned) group) & 1))))
        return fail(std::string(fn) + ": unsupported ConvRot group size (0, or a power of 4 at most 256 dividing K)");
    if (!x || !q || !s) return fail(std::string(fn) + ": x, q and s are required");
    if (!aligned16(x) || !aligned16(q)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return launch_quantize(c, x, x_dt, M, K, group, q, s);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_swiglu_quant(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, int h_dt, int rot, int group,
                                int8_t* q, float* s) try {
    if (M <= 0 || C <= 0) return 0;
    const char* fn = "h3s_swiglu_quant";
    if (!dt_ok(x_dt) || !dt_ok(h_dt)) return fail(std::string(fn) + ": unknown element type");
    const int V = vec_of(x_dt);
    if (C % V != 0) return fail(std::string(fn) + ": C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors per row)");
    if (!x || !q || !s) return fail(std::string(fn) + ": x, q and s are required");
    if (!aligned16(x) || !aligned16(q)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    if (rot_checks(fn, rot, group, C, V)) return -1;
    const RowPlan p = row_plan(C / V);
    if (!p.L) return fail(std::string(fn) + too_long);
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    const QuantArgs A{x, M, C, nullptr, 0.0f, nullptr, nullptr, nullptr, H3S_F32, h_dt, rot,
                      rot != H3S_ROT_NONE ? group : 0, rot != H3S_ROT_NONE ? inv_sqrt_group(group) : 1.0f, q, s};
    return dispatch(c, fn, x_dt, A, QUANT_SWIGLU, p);
} catch (const std::exception& e) { return fail(e.what()); }

namespace h3 {
static int rot_checks(const char* fn, int rot, int group, int64_t C, int V) {
    // a group of G features spans G / V lanes of one wavefront
    if (rot == H3S_ROT_SYLVESTER) {
        if (!is_pow2(group) || group < 2 || group > 64 * V || C % group != 0)
            return fail(std::string(fn) + ": a Sylvester group is a power of 2 dividing C, at most " + std::to_string(64 * V));
    } else if (rot == H3S_ROT_REGULAR) {
        if (!is_pow2(group) || (__builtin_ctz((unsigned) group) & 1) || group < 4 || group > 256 || C % group != 0)
            return fail(std::string(fn) + ": a regular group is a power of 4 dividing C, at most 256");
    } else if (rot != H3S_ROT_NONE) return fail(std::string(fn) + ": unknown rotation");
    return 0;
}
}  // namespace h3
