// rownorm.hip - the row-norm entry points: h3s_rms_norm_mod, h3s_layer_norm (kernels/h3sycl.cpp:766-810,
// 1248-1274) and the fused h3s_norm_mod_act_gate. All three are the row chain kernel of chain_impl.h: one pass over
// each row, every input read once, every output written once.
#include "chain_impl.h"

namespace h3 {

template <int XDT> int chain_launch(Ctx*, const char*, const ChainArgs&, RowPlan);
extern template int chain_launch<H3S_BF16>(Ctx*, const char*, const ChainArgs&, RowPlan);
extern template int chain_launch<H3S_F16>(Ctx*, const char*, const ChainArgs&, RowPlan);
extern template int chain_launch<H3S_F32>(Ctx*, const char*, const ChainArgs&, RowPlan);

// the checks every row chain shares: element types, whole 16-byte vectors per row, alignment, row length
static int chain_checks(const char* fn, const ChainArgs& A, int x_dt, std::initializer_list<int> dts, RowPlan* p) {
    for (int d : dts)
        if (!dt_ok(d)) return fail(std::string(fn) + ": unknown element type");
    if (!dt_ok(x_dt)) return fail(std::string(fn) + ": unknown element type");
    const int V = vec_of(x_dt);
    if (A.C % V != 0)
        return fail(std::string(fn) + ": C must be a multiple of " + std::to_string(V) + " (whole 16-byte vectors per row)");
    for (const void* q : {A.x, (const void*) A.w, (const void*) A.b, A.scale, A.shift, A.gate, A.res, (const void*) A.out})
        if (q && !aligned16(q)) return fail(std::string(fn) + ": tensors must be 16-byte aligned");
    if (!A.x || !A.out) return fail(std::string(fn) + ": x and out are required");
    *p = row_plan(A.C / V);
    if (!p->L)
        return fail(std::string(fn) + ": rows longer than 2048 16-byte vectors (16384 16-bit or 8192 float32 features) are not supported");
    return 0;
}

static int chain_dispatch(Ctx* c, const char* fn, int x_dt, const ChainArgs& A, RowPlan p) {
    switch (x_dt) {
        case H3S_BF16: return chain_launch<H3S_BF16>(c, fn, A, p);
        case H3S_F16: return chain_launch<H3S_F16>(c, fn, A, p);
        default: return chain_launch<H3S_F32>(c, fn, A, p);
    }
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_rms_norm_mod(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps,
                                const int32_t* rows, const float* scale, const float* shift, void* out, int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    const char* fn = "h3s_rms_norm_mod";
    const bool mod = rows && scale && shift;   // kernels/h3sycl.cpp:787-810: modulation only with all three
    const ChainArgs A{x, M, C, H3S_NORM_RMS, weight, nullptr, eps, mod ? rows : nullptr, mod ? scale : nullptr,
                      mod ? shift : nullptr, nullptr, H3S_F32, H3S_ACT_NONE, nullptr, H3S_F32, out, out_dt};
    RowPlan p;
    if (chain_checks(fn, A, x_dt, {out_dt}, &p)) return -1;
    if (!weight) return fail(std::string(fn) + ": the weight is required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    // the model's hidden width: one wavefront a row (the same arithmetic and order; the chain's four wavefronts a
    // row leave three eighths of their last chunk slot idle at 5376 features)
    const int r = launch_norm_out(c, fn, x, x_dt, M, C, weight, eps, A.rows, A.scale ? (const float*) A.scale : nullptr,
                                  A.shift ? (const float*) A.shift : nullptr, out, out_dt);
    if (r != 1) return r;
    return chain_dispatch(c, fn, x_dt, A, p);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_layer_norm(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, const float* bias,
                              float eps, void* out, int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    const char* fn = "h3s_layer_norm";
    const ChainArgs A{x, M, C, H3S_NORM_LAYER, weight, bias, eps, nullptr, nullptr, nullptr, nullptr, H3S_F32,
                      H3S_ACT_NONE, nullptr, H3S_F32, out, out_dt};
    RowPlan p;
    if (chain_checks(fn, A, x_dt, {out_dt}, &p)) return -1;
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return chain_dispatch(c, fn, x_dt, A, p);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_norm_mod_act_gate(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, int norm, const float* weight,
                                     const float* bias, float eps, const int32_t* rows, const void* scale, const void* shift,
                                     const void* gate, int tab_dt, int act, const void* res, int res_dt, void* out,
                                     int out_dt) try {
    if (M <= 0 || C <= 0) return 0;
    const char* fn = "h3s_norm_mod_act_gate";
    const bool mod = scale && shift;
    const ChainArgs A{x, M, C, norm, weight, bias, eps, rows, mod ? scale : nullptr, mod ? shift : nullptr, gate, tab_dt, act,
                      res, res_dt, out, out_dt};
    RowPlan p;
    if (chain_checks(fn, A, x_dt, {out_dt, tab_dt, res_dt}, &p)) return -1;
    if (norm != H3S_NORM_RMS && norm != H3S_NORM_LAYER) return fail(std::string(fn) + ": unknown norm");
    if (act != H3S_ACT_NONE && act != H3S_ACT_GELU_TANH && act != H3S_ACT_SILU) return fail(std::string(fn) + ": unknown activation");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return chain_dispatch(c, fn, x_dt, A, p);
} catch (const std::exception& e) { return fail(e.what()); }
